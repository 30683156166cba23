// C ABI entry points: context, device memory, matrices, the linear products,
// device quantization and attention. The decoder entry points are in
// decoder.hip.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include <initializer_list>
#include <mutex>
#include <vector>

#include "common.h"

namespace qwh {

int32_t fail(qwh_ctx *ctx, int32_t status, const char *fmt, ...) {
    if (ctx) {
        char buf[512];
        va_list args;
        va_start(args, fmt);
        vsnprintf(buf, sizeof buf, fmt, args);
        va_end(args);
        ctx->last_error = buf;
    }
    return status;
}

int32_t check_hip(qwh_ctx *ctx, hipError_t err, const char *what) {
    if (err == hipSuccess) return QWH_OK;
    (void)hipGetLastError();
    return fail(ctx, QWH_E_DEVICE, "%s: %s (%d)", what, hipGetErrorString(err), (int)err);
}

int32_t ensure_workspace(qwh_ctx *ctx, Workspace &ws, size_t bytes) {
    if (ws.bytes >= bytes) return QWH_OK;
    if (ws.ptr) {
        // Work already queued may still read the old buffer.
        QWH_TRY(check_hip(ctx, hipStreamSynchronize(ctx->stream), "workspace sync"));
        (void)hipFree(ws.ptr);
        ws.ptr = nullptr;
        ws.bytes = 0;
    }
    const size_t rounded = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    const hipError_t err = hipMalloc(&ws.ptr, rounded);
    if (err != hipSuccess) {
        (void)hipGetLastError();
        ws.ptr = nullptr;
        return fail(ctx, QWH_E_OUT_OF_MEMORY, "workspace of %zu bytes: %s", rounded, hipGetErrorString(err));
    }
    ws.bytes = rounded;
    return QWH_OK;
}

const Matrix *find_matrix(qwh_ctx *ctx, uint64_t handle) {
    auto it = ctx->matrices.find(handle);
    return it == ctx->matrices.end() ? nullptr : &it->second;
}

namespace {

bool is_quant_format(int32_t format) {
    return format == QWH_FORMAT_Q4 || format == QWH_FORMAT_Q5 || format == QWH_FORMAT_Q8;
}

int32_t check_device_ptr(qwh_ctx *ctx, const void *p, const char *what) {
    if (!p) return fail(ctx, QWH_E_INVALID_ARGUMENT, "%s is null", what);
    return QWH_OK;
}

// Plane sizes of a rows x cols matrix (quant.zig:77-99).
int32_t plane_sizes(qwh_ctx *ctx, int32_t format, uint32_t rows, uint32_t cols, size_t &scales, size_t &data) {
    if (!is_quant_format(format)) return fail(ctx, QWH_E_UNSUPPORTED, "format %d is not quantized", format);
    if (cols == 0 || cols % kGroup != 0)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "cols %u is not a whole number of groups of 64", cols);
    const size_t groups = (size_t)rows * (cols / kGroup);
    scales = groups * 2;
    data = groups * (size_t)data_bytes_per_group(format);
    return QWH_OK;
}

// Plane sizes of any matrix: the quantized planes above, or for f32 / f16
// (kernels.zig:160-166 Matrix .f32 / .f16) no scale plane and rows * cols
// elements.
int32_t matrix_bytes(qwh_ctx *ctx, int32_t format, uint32_t rows, uint32_t cols, size_t &scales, size_t &data) {
    if (!is_dense_format(format)) return plane_sizes(ctx, format, rows, cols, scales, data);
    // Matrix.rows divides the element count by cols (kernels.zig:170-172).
    if (cols == 0) return fail(ctx, QWH_E_SHAPE_MISMATCH, "cols is 0");
    scales = 0;
    data = (size_t)rows * cols * dense_element_bytes(format);
    return QWH_OK;
}

}  // namespace

uint64_t add_matrix(qwh_ctx *ctx, const Matrix &m) {
    const uint64_t handle = ctx->next_handle++;
    ctx->matrices[handle] = m;
    return handle;
}

}  // namespace qwh

using namespace qwh;

// Device scratch of the allocation-free decode attention
// (qwh_decode_attention_q8_noalloc): the per-range softmax records (m, l,
// acc) that the range kernel writes and the merge kernel reads. Every GPU the
// library runs on holds its own copy until the process ends. In host code the
// name is only a handle for hipGetSymbolAddress: kernels and copies use the
// per-device address it resolves (scratch_address below).
constexpr size_t kNoAllocScratchBytes = 8u << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void *g_scratch_address[kMaxDevices] = {};

// Resolves this device's copy of `scratch`, once per device, with that device
// current (tried by qwh_create after hipSetDevice; a failure there is
// recorded only by the no-alloc entry point, which tries again).
int32_t resolve_scratch(int device) {
    if (device < 0 || device >= kMaxDevices) return QWH_E_UNSUPPORTED;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_address[device]) return QWH_OK;
    void *ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !ptr) {
        (void)hipGetLastError();
        return QWH_E_DEVICE;
    }
    g_scratch_address[device] = ptr;
    return QWH_OK;
}

void *scratch_address(int device) {
    if (device < 0 || device >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    return g_scratch_address[device];
}

}  // namespace

extern "C" {

int32_t qwh_abi_version(void) { return QWH_ABI_VERSION; }

const char *qwh_status_string(int32_t status) {
    switch (status) {
    case QWH_OK: return "ok";
    case QWH_E_INVALID_ARGUMENT: return "invalid_argument";
    case QWH_E_OUT_OF_MEMORY: return "out_of_memory";
    case QWH_E_UNSUPPORTED: return "unsupported";
    case QWH_E_SHAPE_MISMATCH: return "shape_mismatch";
    case QWH_E_INVALID_STATE: return "invalid_state";
    case QWH_E_LIMIT_EXCEEDED: return "limit_exceeded";
    case QWH_E_NOT_FOUND: return "not_found";
    case QWH_E_BAD_MAGIC: return "bad_magic";
    case QWH_E_BAD_VERSION: return "bad_version";
    case QWH_E_CHECKSUM_MISMATCH: return "checksum_mismatch";
    case QWH_E_TRUNCATED: return "truncated";
    case QWH_E_UNSUPPORTED_MODEL: return "unsupported_model";
    case QWH_E_DEVICE: return "device";
    default: return "unknown";
    }
}

int32_t qwh_create(uint32_t device_index, qwh_ctx **out) {
    if (!out) return QWH_E_INVALID_ARGUMENT;
    *out = nullptr;
    int count = 0;
    hipError_t err = hipGetDeviceCount(&count);
    if (err != hipSuccess || count == 0) {
        (void)hipGetLastError();
        return QWH_E_DEVICE;
    }
    if ((int)device_index >= count) return QWH_E_INVALID_ARGUMENT;
    if (hipSetDevice((int)device_index) != hipSuccess) return QWH_E_DEVICE;
    qwh_ctx *ctx = new qwh_ctx();
    ctx->device = (int)device_index;
    hipDeviceProp_t prop{};
    if (hipGetDeviceProperties(&prop, ctx->device) == hipSuccess) ctx->cus = prop.multiProcessorCount;
    if (ctx->cus <= 0) ctx->cus = 256;
    if (hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking) != hipSuccess) {
        delete ctx;
        return QWH_E_DEVICE;
    }
    // The device's copy of the allocation-free entry point's scratch. Only
    // that entry point needs it: it reports a failure itself.
    (void)resolve_scratch(ctx->device);
    for (auto &e : ctx->events) {
        if (hipEventCreate(&e) != hipSuccess) {
            qwh_destroy(ctx);
            return QWH_E_DEVICE;
        }
    }
    *out = ctx;
    return QWH_OK;
}

int32_t qwh_destroy(qwh_ctx *ctx) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (auto &kv : ctx->matrices) {
        if (kv.second.owned) {
            (void)hipFree(kv.second.scales);
            (void)hipFree(kv.second.data);
        }
    }
    for (auto &kv : ctx->shards) (void)hipFree(kv.second.payload);
    for (auto &e : ctx->events)
        if (e) (void)hipEventDestroy(e);
    if (ctx->digits.ptr) (void)hipFree(ctx->digits.ptr);
    if (ctx->scratch.ptr) (void)hipFree(ctx->scratch.ptr);
    if (ctx->audio.ptr) (void)hipFree(ctx->audio.ptr);
    if (ctx->front.ptr) (void)hipFree(ctx->front.ptr);
    if (ctx->front_table.ptr) (void)hipFree(ctx->front_table.ptr);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return QWH_OK;
}

int32_t qwh_sync(qwh_ctx *ctx) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    return check_hip(ctx, hipStreamSynchronize(ctx->stream), "sync");
}

const char *qwh_last_error(qwh_ctx *ctx) { return ctx ? ctx->last_error.c_str() : ""; }

int32_t qwh_device_cus(qwh_ctx *ctx, uint32_t *out) {
    if (!ctx || !out) return QWH_E_INVALID_ARGUMENT;
    *out = (uint32_t)ctx->cus;
    return QWH_OK;
}

int32_t qwh_alloc(qwh_ctx *ctx, uint64_t bytes, void **out_dev) {
    if (!ctx || !out_dev) return QWH_E_INVALID_ARGUMENT;
    *out_dev = nullptr;
    const hipError_t err = hipMalloc(out_dev, bytes ? bytes : 1);
    if (err != hipSuccess) {
        (void)hipGetLastError();
        *out_dev = nullptr;
        return fail(ctx, QWH_E_OUT_OF_MEMORY, "hipMalloc(%llu): %s", (unsigned long long)bytes, hipGetErrorString(err));
    }
    return QWH_OK;
}

int32_t qwh_free(qwh_ctx *ctx, void *dev) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    if (!dev) return QWH_OK;
    QWH_TRY(check_hip(ctx, hipStreamSynchronize(ctx->stream), "free sync"));
    return check_hip(ctx, hipFree(dev), "free");
}

int32_t qwh_upload(qwh_ctx *ctx, void *dst_dev, const void *src, uint64_t bytes) {
    if (!ctx || (!bytes ? false : (!dst_dev || !src))) return QWH_E_INVALID_ARGUMENT;
    if (!bytes) return QWH_OK;
    // The source is pageable host memory the caller may reuse on return:
    // copy synchronously with respect to the host.
    QWH_TRY(check_hip(ctx, hipMemcpyAsync(dst_dev, src, bytes, hipMemcpyHostToDevice, ctx->stream), "upload"));
    return check_hip(ctx, hipStreamSynchronize(ctx->stream), "upload sync");
}

int32_t qwh_download(qwh_ctx *ctx, void *dst, const void *src_dev, uint64_t bytes) {
    if (!ctx || (!bytes ? false : (!dst || !src_dev))) return QWH_E_INVALID_ARGUMENT;
    if (!bytes) return QWH_OK;
    QWH_TRY(check_hip(ctx, hipMemcpyAsync(dst, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream), "download"));
    return check_hip(ctx, hipStreamSynchronize(ctx->stream), "download sync");
}

int32_t qwh_memset(qwh_ctx *ctx, void *dst_dev, int32_t value, uint64_t bytes) {
    if (!ctx || (bytes && !dst_dev)) return QWH_E_INVALID_ARGUMENT;
    return check_hip(ctx, hipMemsetAsync(dst_dev, value, bytes, ctx->stream), "memset");
}

int32_t qwh_stream_read(qwh_ctx *ctx, const void *src_dev, uint64_t bytes, uint32_t blocks_per_cu, uint32_t *sink_dev) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    if (bytes == 0) return QWH_OK;
    QWH_TRY(check_device_ptr(ctx, src_dev, "src"));
    QWH_TRY(check_device_ptr(ctx, sink_dev, "sink"));
    if (((uintptr_t)src_dev & 15u) || (bytes & 15u))
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "src and bytes must be 16-byte aligned");
    if (blocks_per_cu == 0 || blocks_per_cu > 8)
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "blocks_per_cu %u outside 1..8", blocks_per_cu);
    return check_hip(ctx, launch_stream_read(ctx->stream, ctx->cus, src_dev, bytes, blocks_per_cu, sink_dev),
                     "stream read");
}

int32_t qwh_event_record(qwh_ctx *ctx, uint32_t slot) {
    if (!ctx || slot >= (uint32_t)kMaxEvents) return QWH_E_INVALID_ARGUMENT;
    return check_hip(ctx, hipEventRecord(ctx->events[slot], ctx->stream), "event record");
}

int32_t qwh_event_elapsed(qwh_ctx *ctx, uint32_t start, uint32_t end, float *out_ms) {
    if (!ctx || !out_ms || start >= (uint32_t)kMaxEvents || end >= (uint32_t)kMaxEvents) return QWH_E_INVALID_ARGUMENT;
    QWH_TRY(check_hip(ctx, hipEventSynchronize(ctx->events[end]), "event sync"));
    return check_hip(ctx, hipEventElapsedTime(out_ms, ctx->events[start], ctx->events[end]), "event elapsed");
}

int32_t qwh_matrix_upload(qwh_ctx *ctx, int32_t format, uint32_t rows, uint32_t cols, const uint8_t *scales,
                          uint64_t scales_len, const uint8_t *data, uint64_t data_len, uint64_t *out_matrix) {
    const bool dense = is_dense_format(format);
    if (!ctx || !out_matrix || (!scales && !dense) || !data) return QWH_E_INVALID_ARGUMENT;
    size_t s_bytes, d_bytes;
    QWH_TRY(matrix_bytes(ctx, format, rows, cols, s_bytes, d_bytes));
    if (scales_len != s_bytes)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "scale plane is %llu bytes, a %ux%u matrix needs %zu",
                    (unsigned long long)scales_len, rows, cols, s_bytes);
    if (data_len != d_bytes)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "data plane is %llu bytes, a %ux%u matrix needs %zu",
                    (unsigned long long)data_len, rows, cols, d_bytes);
    Matrix m;
    m.format = format;
    m.rows = rows;
    m.cols = cols;
    m.owned = true;
    if ((!dense && hipMalloc(&m.scales, s_bytes ? s_bytes : 1) != hipSuccess) ||
        hipMalloc(&m.data, d_bytes ? d_bytes : 1) != hipSuccess) {
        (void)hipGetLastError();
        if (m.scales) (void)hipFree(m.scales);
        return fail(ctx, QWH_E_OUT_OF_MEMORY, "matrix planes of %zu + %zu bytes", s_bytes, d_bytes);
    }
    int32_t st = QWH_OK;
    if (s_bytes)
        st = check_hip(ctx, hipMemcpyAsync(m.scales, scales, s_bytes, hipMemcpyHostToDevice, ctx->stream), "upload scales");
    if (st == QWH_OK)
        st = check_hip(ctx, hipMemcpyAsync(m.data, data, d_bytes, hipMemcpyHostToDevice, ctx->stream), "upload data");
    if (st == QWH_OK) st = check_hip(ctx, hipStreamSynchronize(ctx->stream), "upload sync");
    if (st != QWH_OK) {
        (void)hipFree(m.scales);
        (void)hipFree(m.data);
        return st;
    }
    *out_matrix = add_matrix(ctx, m);
    return QWH_OK;
}

int32_t qwh_matrix_wrap(qwh_ctx *ctx, int32_t format, uint32_t rows, uint32_t cols, const void *scales_dev,
                        const void *data_dev, uint64_t *out_matrix) {
    if (!ctx || !out_matrix) return QWH_E_INVALID_ARGUMENT;
    size_t s_bytes, d_bytes;
    QWH_TRY(matrix_bytes(ctx, format, rows, cols, s_bytes, d_bytes));
    QWH_TRY(check_device_ptr(ctx, data_dev, "data"));
    if (is_dense_format(format)) {
        // model.zig:79-90 Binding f32Values / f16Values: element-aligned.
        if (((uintptr_t)data_dev & (dense_element_bytes(format) - 1)) != 0)
            return fail(ctx, QWH_E_INVALID_ARGUMENT, "f32 / f16 elements must be aligned to their size");
        scales_dev = nullptr;
    } else {
        QWH_TRY(check_device_ptr(ctx, scales_dev, "scales"));
        if (((uintptr_t)data_dev & 15u) != 0)
            return fail(ctx, QWH_E_INVALID_ARGUMENT, "data plane must be 16-byte aligned (quant.zig:61-63)");
        if (((uintptr_t)scales_dev & 1u) != 0)
            return fail(ctx, QWH_E_INVALID_ARGUMENT, "scale plane must be 2-byte aligned");
    }
    Matrix m;
    m.format = format;
    m.rows = rows;
    m.cols = cols;
    m.scales = static_cast<uint8_t *>(const_cast<void *>(scales_dev));
    m.data = static_cast<uint8_t *>(const_cast<void *>(data_dev));
    m.owned = false;
    *out_matrix = add_matrix(ctx, m);
    return QWH_OK;
}

int32_t qwh_matrix_synthetic(qwh_ctx *ctx, int32_t format, uint32_t rows, uint32_t cols, uint32_t seed, uint32_t stream,
                             float value_scale, uint64_t *out_matrix) {
    if (!ctx || !out_matrix) return QWH_E_INVALID_ARGUMENT;
    size_t s_bytes, d_bytes;
    QWH_TRY(matrix_bytes(ctx, format, rows, cols, s_bytes, d_bytes));
    const bool dense = is_dense_format(format);
    Matrix m;
    m.format = format;
    m.rows = rows;
    m.cols = cols;
    m.owned = true;
    if ((!dense && hipMalloc(&m.scales, s_bytes ? s_bytes : 1) != hipSuccess) ||
        hipMalloc(&m.data, d_bytes ? d_bytes : 1) != hipSuccess) {
        (void)hipGetLastError();
        if (m.scales) (void)hipFree(m.scales);
        return fail(ctx, QWH_E_OUT_OF_MEMORY, "matrix planes of %zu + %zu bytes", s_bytes, d_bytes);
    }
    // f32 values go straight into the data plane; f16 and quantized ones
    // through a slab of f32 values.
    const size_t slab_values = (size_t)64 << 20;
    float *temp = nullptr;
    int32_t st = format == QWH_FORMAT_F32 ? QWH_OK : check_hip(ctx, hipMalloc(&temp, slab_values * 4), "synthetic temp");
    const uint32_t slab_rows = (uint32_t)(slab_values / cols) ? (uint32_t)(slab_values / cols) : 1;
    const size_t gpr = cols / kGroup;
    const int db = data_bytes_per_group(format);
    for (uint32_t r = 0; r < rows && st == QWH_OK; r += slab_rows) {
        const uint32_t n = rows - r < slab_rows ? rows - r : slab_rows;
        const uint64_t first = (uint64_t)r * cols, count = (uint64_t)n * cols;
        float *values = format == QWH_FORMAT_F32 ? reinterpret_cast<float *>(m.data) + first : temp;
        st = check_hip(ctx, launch_synth_normal(ctx->stream, seed, stream, first, count, value_scale, values),
                       "synthetic values");
        if (st != QWH_OK || format == QWH_FORMAT_F32) continue;
        if (format == QWH_FORMAT_F16)
            st = check_hip(ctx, launch_f32_to_f16(ctx->stream, temp, count, reinterpret_cast<uint16_t *>(m.data) + first),
                           "f16 values");
        else
            st = check_hip(ctx, launch_quantize_rows(ctx->stream, format, temp, (uint64_t)n * gpr,
                                                     m.scales + (size_t)r * gpr * 2, m.data + (size_t)r * gpr * db),
                           "quantize");
    }
    if (st == QWH_OK) st = check_hip(ctx, hipStreamSynchronize(ctx->stream), "synthetic sync");
    if (temp) (void)hipFree(temp);
    if (st != QWH_OK) {
        (void)hipFree(m.scales);
        (void)hipFree(m.data);
        return st;
    }
    *out_matrix = add_matrix(ctx, m);
    return QWH_OK;
}

int32_t qwh_matrix_planes(qwh_ctx *ctx, uint64_t matrix, void **scales_dev, void **data_dev) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    const Matrix *m = find_matrix(ctx, matrix);
    if (!m) return fail(ctx, QWH_E_NOT_FOUND, "unknown matrix handle %llu", (unsigned long long)matrix);
    if (scales_dev) *scales_dev = m->scales;
    if (data_dev) *data_dev = m->data;
    return QWH_OK;
}

int32_t qwh_matrix_release(qwh_ctx *ctx, uint64_t matrix) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    auto it = ctx->matrices.find(matrix);
    if (it == ctx->matrices.end()) return fail(ctx, QWH_E_NOT_FOUND, "unknown matrix handle %llu", (unsigned long long)matrix);
    if (it->second.owned) {
        QWH_TRY(check_hip(ctx, hipStreamSynchronize(ctx->stream), "release sync"));
        (void)hipFree(it->second.scales);
        (void)hipFree(it->second.data);
    }
    ctx->matrices.erase(it);
    return QWH_OK;
}

int32_t qwh_linear(qwh_ctx *ctx, uint64_t matrix, const float *x_dev, uint32_t cols, uint32_t tokens, float *out_dev) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    const Matrix *m = find_matrix(ctx, matrix);
    if (!m) return fail(ctx, QWH_E_NOT_FOUND, "unknown matrix handle %llu", (unsigned long long)matrix);
    // kernels.zig:129-139 shape checks.
    if (cols != m->cols) return fail(ctx, QWH_E_SHAPE_MISMATCH, "x has %u columns, the matrix %u", cols, m->cols);
    if (tokens == 0) return QWH_OK;
    if (tokens > 65535) return fail(ctx, QWH_E_LIMIT_EXCEEDED, "tokens %u > 65535", tokens);
    QWH_TRY(check_device_ptr(ctx, x_dev, "x"));
    QWH_TRY(check_device_ptr(ctx, out_dev, "out"));
    if (((uintptr_t)x_dev & 15u) != 0) return fail(ctx, QWH_E_INVALID_ARGUMENT, "x must be 16-byte aligned");
    if (m->rows == 0) return QWH_OK;
    if (m->format == QWH_FORMAT_Q4) {
        if (tokens >= 2) {
            // Several tokens: int8 digit planes, then one matrix-core pass
            // over the weights per 16 tokens.
            GemvInput in;
            in.mode = GemvInput::F32;
            in.x = x_dev;
            QWH_TRY(ensure_workspace(ctx, ctx->digits, batch_digit_bytes(tokens, cols)));
            const size_t parts = batch_partial_bytes(tokens, *m);
            if (parts) QWH_TRY(ensure_workspace(ctx, ctx->scratch, parts));
            QWH_TRY(check_hip(ctx, launch_prep_batch(ctx->stream, in, tokens, cols, ctx->digits.ptr), "prep batch"));
            return check_hip(ctx, launch_gemv_batch(ctx->stream, ctx->digits.ptr, *m, tokens, out_dev, nullptr,
                                                       false, static_cast<float *>(ctx->scratch.ptr)),
                             "gemv q4 batch");
        }
        if (gemv_q4_fused_supported(m->rows, m->cols)) {
            // One kernel: each wavefront encodes its own activations.
            GemvInput in;
            in.mode = GemvInput::F32;
            in.x = x_dev;
            return check_hip(ctx, launch_gemv_q4_src(ctx->stream, ctx->cus, in, *m, tokens, out_dev, nullptr), "gemv q4");
        }
        QWH_TRY(ensure_workspace(ctx, ctx->digits, q4_digit_bytes(tokens, cols)));
        QWH_TRY(check_hip(ctx, launch_prep_q4(ctx->stream, x_dev, tokens, cols, ctx->digits.ptr), "prep q4"));
        return check_hip(ctx, launch_gemv_q4(ctx->stream, ctx->cus, ctx->digits.ptr, *m, tokens, out_dev, nullptr), "gemv q4");
    }
    if (m->format == QWH_FORMAT_Q8) {
        if (tokens >= 2) {
            // Several tokens: the q4 path's int8 digit planes and one
            // matrix-core pass over the codes per 16 tokens (u - 128 is
            // already a signed byte), so W streams once, not once per token.
            if (((uintptr_t)m->data & 15u) != 0)
                return fail(ctx, QWH_E_INVALID_ARGUMENT, "q8 data plane must be 16-byte aligned");
            GemvInput in;
            in.mode = GemvInput::F32;
            in.x = x_dev;
            QWH_TRY(ensure_workspace(ctx, ctx->digits, batch_digit_bytes(tokens, cols)));
            const size_t parts = batch_partial_bytes(tokens, *m);
            if (parts) QWH_TRY(ensure_workspace(ctx, ctx->scratch, parts));
            QWH_TRY(check_hip(ctx, launch_prep_batch(ctx->stream, in, tokens, cols, ctx->digits.ptr), "prep batch"));
            return check_hip(ctx, launch_gemv_batch(ctx->stream, ctx->digits.ptr, *m, tokens, out_dev, nullptr, false,
                                                    static_cast<float *>(ctx->scratch.ptr)),
                             "gemv q8 batch");
        }
        return check_hip(ctx, launch_gemv_q8(ctx->stream, ctx->cus, x_dev, *m, tokens, out_dev, nullptr), "gemv q8");
    }
    if (m->format == QWH_FORMAT_Q5) {
        if (((uintptr_t)m->data & 7u) != 0)
            return fail(ctx, QWH_E_INVALID_ARGUMENT, "q5 data plane must be 8-byte aligned");
        if (tokens >= 2 && gemv_batch_supported(*m)) {
            // Several tokens (K a multiple of 256): the int8 digit planes and
            // one matrix-core pass over the codes per 16 tokens.
            GemvInput in;
            in.mode = GemvInput::F32;
            in.x = x_dev;
            QWH_TRY(ensure_workspace(ctx, ctx->digits, batch_digit_bytes(tokens, cols)));
            const size_t parts = batch_partial_bytes(tokens, *m);
            if (parts) QWH_TRY(ensure_workspace(ctx, ctx->scratch, parts));
            QWH_TRY(check_hip(ctx, launch_prep_batch(ctx->stream, in, tokens, cols, ctx->digits.ptr), "prep batch"));
            return check_hip(ctx, launch_gemv_batch(ctx->stream, ctx->digits.ptr, *m, tokens, out_dev, nullptr, false,
                                                    static_cast<float *>(ctx->scratch.ptr)),
                             "gemv q5 batch");
        }
        if (!gemv_b8_supported(m->format, m->rows, m->cols))
            return fail(ctx, QWH_E_UNSUPPORTED, "q5 linear is built for K <= 6144 and data planes below 4 GiB");
        GemvInput in;
        in.mode = GemvInput::F32;
        in.x = x_dev;
        return check_hip(ctx, launch_gemv_b8(ctx->stream, ctx->cus, in, *m, tokens, out_dev, nullptr), "gemv q5");
    }
    if (is_dense_format(m->format)) {
        // kernels.zig:54-112 linearF32 / linearF16: up to four tokens per
        // pass over the weights.
        if (!gemv_dense_supported(m->format, m->cols))
            return fail(ctx, QWH_E_UNSUPPORTED, "f32 / f16 linear is built for rows of at most %u values", kDenseMaxCols);
        GemvInput in;
        in.mode = GemvInput::F32;
        in.x = x_dev;
        return check_hip(ctx, launch_gemv_dense(ctx->stream, ctx->cus, in, *m, tokens, out_dev, nullptr), "gemv dense");
    }
    return fail(ctx, QWH_E_UNSUPPORTED, "linear over format %d is not built", m->format);
}

int32_t qwh_activation_bytes(uint32_t cols, uint32_t tokens, uint64_t *out_bytes) {
    if (!out_bytes) return QWH_E_INVALID_ARGUMENT;
    if (cols == 0 || cols % kGroup != 0) return QWH_E_SHAPE_MISMATCH;
    *out_bytes = q4_digit_bytes(tokens, cols);
    return QWH_OK;
}

int32_t qwh_activation_prepare(qwh_ctx *ctx, const float *x_dev, uint32_t cols, uint32_t tokens, void *prepared_dev) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    if (cols == 0 || cols % kGroup != 0)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "cols %u is not a whole number of groups of 64", cols);
    if (tokens == 0) return QWH_OK;
    if (tokens > 65535) return fail(ctx, QWH_E_LIMIT_EXCEEDED, "tokens %u > 65535", tokens);
    QWH_TRY(check_device_ptr(ctx, x_dev, "x"));
    QWH_TRY(check_device_ptr(ctx, prepared_dev, "prepared"));
    if ((((uintptr_t)x_dev) | ((uintptr_t)prepared_dev)) & 15u)
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "x and prepared must be 16-byte aligned");
    return check_hip(ctx, launch_prep_q4(ctx->stream, x_dev, tokens, cols, prepared_dev), "prepare activations");
}

int32_t qwh_linear_prepared(qwh_ctx *ctx, uint64_t matrix, const void *prepared_dev, uint32_t tokens, float *out_dev) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    const Matrix *m = find_matrix(ctx, matrix);
    if (!m) return fail(ctx, QWH_E_NOT_FOUND, "unknown matrix handle %llu", (unsigned long long)matrix);
    if (m->format != QWH_FORMAT_Q4) return fail(ctx, QWH_E_UNSUPPORTED, "prepared activations feed q4 matrices");
    if (tokens == 0 || m->rows == 0) return QWH_OK;
    if (tokens > 65535) return fail(ctx, QWH_E_LIMIT_EXCEEDED, "tokens %u > 65535", tokens);
    QWH_TRY(check_device_ptr(ctx, prepared_dev, "prepared"));
    QWH_TRY(check_device_ptr(ctx, out_dev, "out"));
    if (((uintptr_t)prepared_dev) & 15u) return fail(ctx, QWH_E_INVALID_ARGUMENT, "prepared must be 16-byte aligned");
    return check_hip(ctx, launch_gemv_q4(ctx->stream, ctx->cus, prepared_dev, *m, tokens, out_dev, nullptr), "gemv q4");
}

int32_t qwh_linear_bf16(qwh_ctx *ctx, uint64_t matrix, const uint16_t *x_dev, uint32_t cols, uint32_t tokens,
                        float *out_dev) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    const Matrix *m = find_matrix(ctx, matrix);
    if (!m) return fail(ctx, QWH_E_NOT_FOUND, "unknown matrix handle %llu", (unsigned long long)matrix);
    if (cols != m->cols) return fail(ctx, QWH_E_SHAPE_MISMATCH, "x has %u columns, the matrix %u", cols, m->cols);
    if (m->format != QWH_FORMAT_Q4 && m->format != QWH_FORMAT_Q5 && m->format != QWH_FORMAT_Q8)
        return fail(ctx, QWH_E_UNSUPPORTED, "bf16 GEMM is built for q4, q5 and q8");
    if (m->format == QWH_FORMAT_Q5 && ((uintptr_t)m->data & 7u) != 0)
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "q5 data plane must be 8-byte aligned");
    if (m->format == QWH_FORMAT_Q8 && ((uintptr_t)m->data & 15u) != 0)
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "q8 data plane must be 16-byte aligned");
    if (tokens == 0 || m->rows == 0) return QWH_OK;
    if (tokens > 65535u * 128u) return fail(ctx, QWH_E_LIMIT_EXCEEDED, "tokens %u", tokens);
    QWH_TRY(check_device_ptr(ctx, x_dev, "x"));
    QWH_TRY(check_device_ptr(ctx, out_dev, "out"));
    if (((uintptr_t)x_dev & 15u) != 0) return fail(ctx, QWH_E_INVALID_ARGUMENT, "x must be 16-byte aligned");
    const size_t scratch = gemm_scratch_bytes(ctx->cus, tokens, *m);
    if (scratch) QWH_TRY(ensure_workspace(ctx, ctx->scratch, scratch));
    return check_hip(ctx, launch_gemm_bf16(ctx->stream, ctx->cus, x_dev, *m, tokens, out_dev, ctx->scratch.ptr),
                     "gemm bf16");
}

int32_t qwh_quantize_rows(qwh_ctx *ctx, int32_t format, const float *values_dev, uint32_t rows, uint32_t cols,
                          uint8_t *scales_dev, uint8_t *data_dev) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    size_t s_bytes, d_bytes;
    QWH_TRY(plane_sizes(ctx, format, rows, cols, s_bytes, d_bytes));
    if (rows == 0) return QWH_OK;
    QWH_TRY(check_device_ptr(ctx, values_dev, "values"));
    QWH_TRY(check_device_ptr(ctx, scales_dev, "scales"));
    QWH_TRY(check_device_ptr(ctx, data_dev, "data"));
    return check_hip(ctx, launch_quantize_rows(ctx->stream, format, values_dev, (uint64_t)rows * (cols / kGroup), scales_dev,
                                               data_dev), "quantize rows");
}

int32_t qwh_synth_normal(qwh_ctx *ctx, uint32_t seed, uint32_t stream, uint64_t count, float value_scale, float *out_dev) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    if (count == 0) return QWH_OK;
    QWH_TRY(check_device_ptr(ctx, out_dev, "out"));
    return check_hip(ctx, launch_synth_normal(ctx->stream, seed, stream, 0, count, value_scale, out_dev), "synth normal");
}

}  // extern "C"

namespace {

// kernels.zig:712-723 shape checks and the kernels' alignment needs for the
// q8 decode attention; fills `a` for launch_decode_attention_q8 (a.batch 0:
// nothing to do).
int32_t attention_q8_args(qwh_ctx *ctx, float *out_dev, const float *query_dev, const uint8_t *k_scales_dev,
                          const uint8_t *k_codes_dev, const uint8_t *v_scales_dev, const uint8_t *v_codes_dev,
                          uint32_t cached, uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t batch,
                          uint64_t scale_stride_bytes, uint64_t code_stride_bytes, AttentionArgs &a) {
    if (head_dim == 0 || head_dim % kGroup != 0)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "head_dim %u is not a multiple of 64", head_dim);
    if (kv_heads == 0 || heads % kv_heads != 0)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "heads %u not a multiple of kv_heads %u", heads, kv_heads);
    if (cached == 0) return fail(ctx, QWH_E_SHAPE_MISMATCH, "no cached positions (softmax of an empty row)");
    a = AttentionArgs{};
    if (batch == 0) return QWH_OK;
    const size_t kv_width = (size_t)kv_heads * head_dim;
    if (batch > 1 && (scale_stride_bytes < (size_t)cached * (kv_width / kGroup) * 2 || code_stride_bytes < (size_t)cached * kv_width))
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "sequence strides smaller than %u cached rows", cached);
    QWH_TRY(check_device_ptr(ctx, out_dev, "out"));
    QWH_TRY(check_device_ptr(ctx, query_dev, "query"));
    QWH_TRY(check_device_ptr(ctx, k_scales_dev, "k_scales"));
    QWH_TRY(check_device_ptr(ctx, k_codes_dev, "k_codes"));
    QWH_TRY(check_device_ptr(ctx, v_scales_dev, "v_scales"));
    QWH_TRY(check_device_ptr(ctx, v_codes_dev, "v_codes"));
    if (((uintptr_t)k_codes_dev | (uintptr_t)v_codes_dev | (uintptr_t)query_dev) & 15u)
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "query and code planes must be 16-byte aligned");
    if (((uintptr_t)k_scales_dev | (uintptr_t)v_scales_dev) & 1u)
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "scale planes must be 2-byte aligned");
    if (batch > 1 && ((scale_stride_bytes & 1u) || (code_stride_bytes & 15u)))
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "sequence strides must keep the plane alignment");
    const uint32_t ratio = heads / kv_heads;
    if (!attention_supported(head_dim, ratio) && !attention_generic_supported(head_dim))
        return fail(ctx, QWH_E_UNSUPPORTED, "attention for head_dim %u is not built", head_dim);
    a.out = out_dev;
    a.query = query_dev;
    // The kernel only reads the cache planes in this form.
    a.k_scales = const_cast<uint8_t *>(k_scales_dev);
    a.k_codes = const_cast<uint8_t *>(k_codes_dev);
    a.v_scales = const_cast<uint8_t *>(v_scales_dev);
    a.v_codes = const_cast<uint8_t *>(v_codes_dev);
    a.cached = cached;
    a.cached_dev = nullptr;
    a.capacity = cached;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    a.batch = batch;
    a.scale_stride = scale_stride_bytes;
    a.code_stride = code_stride_bytes;
    return QWH_OK;
}

}  // namespace

extern "C" {

int32_t qwh_decode_attention_q8(qwh_ctx *ctx, float *out_dev, const float *query_dev, const uint8_t *k_scales_dev,
                                const uint8_t *k_codes_dev, const uint8_t *v_scales_dev, const uint8_t *v_codes_dev,
                                uint32_t cached, uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t batch,
                                uint64_t scale_stride_bytes, uint64_t code_stride_bytes) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    AttentionArgs a;
    QWH_TRY(attention_q8_args(ctx, out_dev, query_dev, k_scales_dev, k_codes_dev, v_scales_dev, v_codes_dev, cached,
                              heads, kv_heads, head_dim, batch, scale_stride_bytes, code_stride_bytes, a));
    if (a.batch == 0) return QWH_OK;
    QWH_TRY(ensure_workspace(ctx, ctx->scratch, attention_scratch_bytes(ctx->cus, a)));
    return check_hip(ctx, launch_decode_attention_q8(ctx->stream, ctx->cus, a, ctx->scratch.ptr, ctx->scratch.bytes),
                     "decode attention q8");
}

int32_t qwh_decode_attention_q8_noalloc(qwh_ctx *ctx, float *out_dev, const float *query_dev,
                                        const uint8_t *k_scales_dev, const uint8_t *k_codes_dev,
                                        const uint8_t *v_scales_dev, const uint8_t *v_codes_dev, uint32_t cached,
                                        uint32_t heads, uint32_t kv_heads, uint32_t head_dim, uint32_t batch,
                                        uint64_t scale_stride_bytes, uint64_t code_stride_bytes) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    AttentionArgs a;
    QWH_TRY(attention_q8_args(ctx, out_dev, query_dev, k_scales_dev, k_codes_dev, v_scales_dev, v_codes_dev, cached,
                              heads, kv_heads, head_dim, batch, scale_stride_bytes, code_stride_bytes, a));
    if (a.batch == 0) return QWH_OK;
    const size_t need = attention_scratch_bytes(ctx->cus, a);
    if (need > kNoAllocScratchBytes)
        return fail(ctx, QWH_E_LIMIT_EXCEEDED, "attention records need %zu bytes; the static scratch holds %zu", need,
                    kNoAllocScratchBytes);
    void *ptr = scratch_address(ctx->device);
    if (!ptr) {
        // Not resolved at qwh_create: once more, with the context's device
        // current.
        if (hipSetDevice(ctx->device) != hipSuccess || resolve_scratch(ctx->device) != QWH_OK) {
            (void)hipGetLastError();
            return fail(ctx, QWH_E_DEVICE, "device %d: the static scratch's address could not be resolved",
                        ctx->device);
        }
        ptr = scratch_address(ctx->device);
    }
    // The records need no clearing: each range writes its record before the
    // merge reads it, and ranges past `cached` are never read.
    return check_hip(ctx, launch_decode_attention_q8(ctx->stream, ctx->cus, a, ptr, kNoAllocScratchBytes),
                     "decode attention q8 (no alloc)");
}

int32_t qwh_decode_attention_f32(qwh_ctx *ctx, float *out_dev, const float *query_dev, const float *keys_dev,
                                 const float *values_dev, uint32_t cached, uint32_t heads, uint32_t kv_heads,
                                 uint32_t head_dim, uint32_t batch, uint64_t stride_bytes) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    // kernels.zig:583-593 shape checks.
    if (head_dim == 0 || kv_heads == 0 || heads % kv_heads != 0)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "heads %u not a multiple of kv_heads %u", heads, kv_heads);
    if (cached == 0) return fail(ctx, QWH_E_SHAPE_MISMATCH, "no cached positions (softmax of an empty row)");
    if (batch == 0) return QWH_OK;
    const size_t kv_width = (size_t)kv_heads * head_dim;
    if (batch > 1 && stride_bytes < (size_t)cached * kv_width * sizeof(float))
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "sequence stride smaller than %u cached rows", cached);
    QWH_TRY(check_device_ptr(ctx, out_dev, "out"));
    QWH_TRY(check_device_ptr(ctx, query_dev, "query"));
    QWH_TRY(check_device_ptr(ctx, keys_dev, "keys"));
    QWH_TRY(check_device_ptr(ctx, values_dev, "values"));
    if (((uintptr_t)keys_dev | (uintptr_t)values_dev | (uintptr_t)query_dev) & 15u)
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "query, keys and values must be 16-byte aligned");
    if (batch > 1 && (stride_bytes & 15u))
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "the sequence stride must keep 16-byte alignment");
    const uint32_t ratio = heads / kv_heads;
    if (!attention_supported(head_dim, ratio) && !attention_generic_supported(head_dim))
        return fail(ctx, QWH_E_UNSUPPORTED, "attention for head_dim %u is not built", head_dim);
    AttentionArgs a{};
    a.out = out_dev;
    a.query = query_dev;
    a.k_codes = reinterpret_cast<uint8_t *>(const_cast<float *>(keys_dev));
    a.v_codes = reinterpret_cast<uint8_t *>(const_cast<float *>(values_dev));
    a.cached = cached;
    a.capacity = cached;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    a.batch = batch;
    a.code_stride = stride_bytes;
    a.f32_cache = true;
    QWH_TRY(ensure_workspace(ctx, ctx->scratch, attention_scratch_bytes(ctx->cus, a)));
    return check_hip(ctx, launch_decode_attention_q8(ctx->stream, ctx->cus, a, ctx->scratch.ptr, ctx->scratch.bytes),
                     "decode attention f32");
}

int32_t qwh_kv_append_q8(qwh_ctx *ctx, const float *key_dev, const float *value_dev, uint32_t kv_width, uint32_t position,
                         uint8_t *k_scales_dev, uint8_t *k_codes_dev, uint8_t *v_scales_dev, uint8_t *v_codes_dev) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    if (kv_width == 0 || kv_width % kGroup != 0)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "kv_width %u is not a multiple of 64", kv_width);
    QWH_TRY(check_device_ptr(ctx, key_dev, "key"));
    QWH_TRY(check_device_ptr(ctx, value_dev, "value"));
    QWH_TRY(check_device_ptr(ctx, k_scales_dev, "k_scales"));
    QWH_TRY(check_device_ptr(ctx, k_codes_dev, "k_codes"));
    QWH_TRY(check_device_ptr(ctx, v_scales_dev, "v_scales"));
    QWH_TRY(check_device_ptr(ctx, v_codes_dev, "v_codes"));
    if (((uintptr_t)k_scales_dev | (uintptr_t)v_scales_dev) & 1u)
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "scale planes must be 2-byte aligned");
    return check_hip(ctx, launch_kv_append_q8(ctx->stream, key_dev, value_dev, kv_width, position, k_scales_dev, k_codes_dev,
                                              v_scales_dev, v_codes_dev), "kv append q8");
}


// ---- audio tower (model.zig:646-735) ----

int32_t qwh_layer_norm(qwh_ctx *ctx, float *out_dev, const float *x_dev, const float *weight_dev,
                       const float *bias_dev, uint32_t width, uint32_t tokens, float eps) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    if (tokens == 0) return QWH_OK;
    if (width == 0) return fail(ctx, QWH_E_SHAPE_MISMATCH, "layer norm over rows of width 0");
    QWH_TRY(check_device_ptr(ctx, out_dev, "out"));
    QWH_TRY(check_device_ptr(ctx, x_dev, "x"));
    QWH_TRY(check_device_ptr(ctx, weight_dev, "weight"));
    QWH_TRY(check_device_ptr(ctx, bias_dev, "bias"));
    return check_hip(ctx, launch_layer_norm(ctx->stream, x_dev, out_dev, weight_dev, bias_dev, width, tokens, eps),
                     "layer norm");
}

int32_t qwh_add_bias(qwh_ctx *ctx, float *x_dev, const float *bias_dev, uint32_t rows, uint32_t tokens) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    if ((uint64_t)rows * tokens == 0) return QWH_OK;
    QWH_TRY(check_device_ptr(ctx, x_dev, "x"));
    QWH_TRY(check_device_ptr(ctx, bias_dev, "bias"));
    return check_hip(ctx, launch_bias_epilogue(ctx->stream, kBiasAdd, x_dev, bias_dev, nullptr, rows, tokens),
                     "add bias");
}

int32_t qwh_gelu(qwh_ctx *ctx, float *x_dev, uint64_t count) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    if (count == 0) return QWH_OK;
    if (count > 0xFFFFFFFFull) return fail(ctx, QWH_E_LIMIT_EXCEEDED, "gelu over %llu values", (unsigned long long)count);
    QWH_TRY(check_device_ptr(ctx, x_dev, "x"));
    return check_hip(ctx, launch_bias_epilogue(ctx->stream, kBiasGelu, x_dev, nullptr, nullptr, (uint32_t)count, 1),
                     "gelu");
}

namespace {

int32_t check_audio_attention(qwh_ctx *ctx, const AudioAttentionArgs &a) {
    QWH_TRY(check_device_ptr(ctx, a.out, "out"));
    QWH_TRY(check_device_ptr(ctx, a.q, "q"));
    QWH_TRY(check_device_ptr(ctx, a.k, "k"));
    QWH_TRY(check_device_ptr(ctx, a.v, "v"));
    if (!audio_attention_supported(a.head_dim))
        return fail(ctx, QWH_E_UNSUPPORTED, "audio attention is built for head_dim 32, 64 and 128, not %u", a.head_dim);
    const uint64_t width = (uint64_t)a.heads * a.head_dim;
    if (a.out_stride < width || a.q_stride < width || a.k_stride < width || a.v_stride < width)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "a row stride is below heads * head_dim = %llu", (unsigned long long)width);
    if ((a.out_stride | a.q_stride | a.k_stride | a.v_stride) & 3u)
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "row strides must be multiples of 4 floats");
    const uintptr_t bits = (uintptr_t)a.out | (uintptr_t)a.q | (uintptr_t)a.k | (uintptr_t)a.v |
                           (uintptr_t)a.q_bias | (uintptr_t)a.k_bias | (uintptr_t)a.v_bias;
    if (bits & 15u) return fail(ctx, QWH_E_INVALID_ARGUMENT, "audio attention buffers must be 16-byte aligned");
    // One workgroup row per window and one layer per head (grid y and z).
    const uint64_t windows = a.window_steps ? ((uint64_t)a.end - a.first + a.window_steps - 1) / a.window_steps : 0;
    if (windows > 65535 || a.heads > 65535)
        return fail(ctx, QWH_E_LIMIT_EXCEEDED, "%llu windows of %u heads: at most 65535 of each",
                    (unsigned long long)windows, a.heads);
    return QWH_OK;
}

}  // namespace

int32_t qwh_audio_attention_window(qwh_ctx *ctx, float *out_dev, uint32_t out_stride, const float *q_dev,
                                   uint32_t q_stride, const float *k_dev, uint32_t k_stride, const float *v_dev,
                                   uint32_t v_stride, uint32_t window_start, uint32_t window_length, uint32_t heads,
                                   uint32_t head_dim) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    if (window_length == 0 || heads == 0) return QWH_OK;
    if ((uint64_t)window_start + window_length > 0xFFFFFFFFull)
        return fail(ctx, QWH_E_LIMIT_EXCEEDED, "window end past 2^32 steps");
    AudioAttentionArgs a;
    a.out = out_dev, a.q = q_dev, a.k = k_dev, a.v = v_dev;
    a.out_stride = out_stride, a.q_stride = q_stride, a.k_stride = k_stride, a.v_stride = v_stride;
    a.first = window_start, a.end = window_start + window_length, a.window_steps = window_length;
    a.heads = heads, a.head_dim = head_dim;
    a.scaling = 1.0f / sqrtf((float)head_dim);
    QWH_TRY(check_audio_attention(ctx, a));
    return check_hip(ctx, launch_audio_attention(ctx->stream, a), "audio attention");
}

int32_t qwh_audio_attention(qwh_ctx *ctx, float *out_dev, uint32_t out_stride, const float *q_dev,
                            const float *k_dev, const float *v_dev, uint32_t qkv_stride, uint32_t steps,
                            uint32_t window_steps, uint32_t heads, uint32_t head_dim) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    if (steps == 0 || heads == 0) return QWH_OK;
    if (window_steps == 0) return fail(ctx, QWH_E_INVALID_ARGUMENT, "window_steps is 0");
    AudioAttentionArgs a;
    a.out = out_dev, a.q = q_dev, a.k = k_dev, a.v = v_dev;
    a.out_stride = out_stride, a.q_stride = a.k_stride = a.v_stride = qkv_stride;
    a.first = 0, a.end = steps, a.window_steps = window_steps;
    a.heads = heads, a.head_dim = head_dim;
    a.scaling = 1.0f / sqrtf((float)head_dim);
    QWH_TRY(check_audio_attention(ctx, a));
    return check_hip(ctx, launch_audio_attention(ctx->stream, a), "audio attention");
}

namespace {

int32_t check_audio_matrix(qwh_ctx *ctx, uint64_t handle, uint32_t rows, uint32_t cols, const char *what) {
    const Matrix *m = find_matrix(ctx, handle);
    if (!m) return fail(ctx, QWH_E_NOT_FOUND, "%s: unknown matrix handle %llu", what, (unsigned long long)handle);
    if (m->rows != rows || m->cols != cols)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "%s is %u x %u, the layer needs %u x %u", what, m->rows, m->cols, rows,
                    cols);
    return QWH_OK;
}

}  // namespace

namespace {

// Several linears over the same activations: for q4 / q8 matrices and two or
// more tokens the digit planes are prepared once and each matrix reads them
// (qwh_linear would prepare them per matrix); q5 goes through qwh_linear one
// by one.
// True when every matrix takes `cols`-wide rows and has a batch GEMV form.
bool batch_ready(qwh_ctx *ctx, std::initializer_list<uint64_t> handles, uint32_t cols) {
    for (uint64_t h : handles) {
        const Matrix *m = find_matrix(ctx, h);
        if (!m || !gemv_batch_supported(*m) || ((uintptr_t)m->data & 15u) != 0 || m->cols != cols || m->rows == 0)
            return false;
    }
    return true;
}

int32_t linear_shared_input(qwh_ctx *ctx, std::initializer_list<uint64_t> handles, const float *x, uint32_t cols,
                            uint32_t tokens, std::initializer_list<float *> outs) {
    const bool shared = tokens >= 2 && ((uintptr_t)x & 15u) == 0 && batch_ready(ctx, handles, cols);
    auto out = outs.begin();
    if (!shared) {
        for (uint64_t h : handles) QWH_TRY(qwh_linear(ctx, h, x, cols, tokens, *out++));
        return QWH_OK;
    }
    size_t parts = 0;
    for (uint64_t h : handles) parts = std::max(parts, batch_partial_bytes(tokens, *find_matrix(ctx, h)));
    QWH_TRY(ensure_workspace(ctx, ctx->digits, batch_digit_bytes(tokens, cols)));
    if (parts) QWH_TRY(ensure_workspace(ctx, ctx->scratch, parts));
    GemvInput in;
    in.mode = GemvInput::F32;
    in.x = x;
    QWH_TRY(check_hip(ctx, launch_prep_batch(ctx->stream, in, tokens, cols, ctx->digits.ptr), "prep batch"));
    for (uint64_t h : handles)
        QWH_TRY(check_hip(ctx, launch_gemv_batch(ctx->stream, ctx->digits.ptr, *find_matrix(ctx, h), tokens, *out++,
                                                    nullptr, false, static_cast<float *>(ctx->scratch.ptr)),
                          "gemv batch"));
    return QWH_OK;
}

// qwh_audio_layer when every linear has a batch GEMV form: the two
// LayerNorms write the GEMVs' activation digits directly, q / k / v read one
// set of digits in one launch, the GELU of ffn_in + bias is applied as
// ffn_out's digits are prepared, and o and ffn_out add their bias and the
// residual stream in their own epilogue (out = encoder + (W x + bias), the
// order of the reference's addBias then addInPlace). Seven launches instead
// of fourteen, and no f32 pass over the normed rows or the projections'
// outputs.
int32_t audio_layer_batch(qwh_ctx *ctx, const qwh_audio_layer_weights *w, float *encoder_dev, uint32_t steps,
                          uint32_t d_model, uint32_t ffn_dim, float eps, const AudioAttentionArgs &a, float *wide) {
    hipStream_t s = ctx->stream;
    size_t parts = 0;
    for (uint64_t h : {w->q, w->k, w->v, w->o, w->ffn_in, w->ffn_out})
        parts = std::max(parts, batch_partial_bytes(steps, *find_matrix(ctx, h)));
    QWH_TRY(ensure_workspace(ctx, ctx->digits,
                             std::max(batch_digit_bytes(steps, d_model), batch_digit_bytes(steps, ffn_dim))));
    if (parts) QWH_TRY(ensure_workspace(ctx, ctx->scratch, parts));
    void *digits = ctx->digits.ptr;
    float *partials = static_cast<float *>(ctx->scratch.ptr);
    auto gemv = [&](uint64_t h, float *out, const float *residual, const float *bias, const char *what) {
        return check_hip(ctx, launch_gemv_batch(s, digits, *find_matrix(ctx, h), steps, out, residual, false, partials,
                                                BatchNorm{}, bias),
                         what);
    };
    // model.zig:657-665 layerNormInto, :765-786 projectQkv (biases join in the attention's loads).
    QWH_TRY(check_hip(ctx, launch_layer_norm_digits(s, encoder_dev, w->attention_norm_weight, w->attention_norm_bias,
                                                    d_model, steps, eps, digits),
                      "audio attention norm"));
    // q, k and v in one launch where their plans agree (one K slice each).
    const Matrix *qkv[3] = {find_matrix(ctx, w->q), find_matrix(ctx, w->k), find_matrix(ctx, w->v)};
    float *const qkv_out[3] = {const_cast<float *>(a.q), const_cast<float *>(a.k), const_cast<float *>(a.v)};
    const hipError_t fused = launch_gemv_batch_multi(s, digits, qkv, qkv_out, 3, steps);
    if (fused == hipErrorNotSupported) {
        QWH_TRY(gemv(w->q, qkv_out[0], nullptr, nullptr, "audio q"));
        QWH_TRY(gemv(w->k, qkv_out[1], nullptr, nullptr, "audio k"));
        QWH_TRY(gemv(w->v, qkv_out[2], nullptr, nullptr, "audio v"));
    } else {
        QWH_TRY(check_hip(ctx, fused, "audio q|k|v"));
    }
    QWH_TRY(check_hip(ctx, launch_audio_attention(s, a), "audio attention"));
    // :824-848 projectAttentionOutput + o bias, :669 addInPlace.
    GemvInput in;
    in.mode = GemvInput::F32;
    in.x = a.out;
    QWH_TRY(check_hip(ctx, launch_prep_batch(s, in, steps, d_model, digits), "audio o prep"));
    QWH_TRY(gemv(w->o, encoder_dev, encoder_dev, w->o_bias, "audio o"));
    // :671-679 layerNormInto, :852-872 activateFfn, :692 addInPlace.
    QWH_TRY(check_hip(ctx, launch_layer_norm_digits(s, encoder_dev, w->final_norm_weight, w->final_norm_bias, d_model,
                                                    steps, eps, digits),
                      "audio final norm"));
    QWH_TRY(gemv(w->ffn_in, wide, nullptr, nullptr, "audio ffn_in"));
    in.x = wide;
    in.gelu_bias = w->ffn_in_bias;
    QWH_TRY(check_hip(ctx, launch_prep_batch(s, in, steps, ffn_dim, digits), "audio ffn prep"));
    return gemv(w->ffn_out, encoder_dev, encoder_dev, w->ffn_out_bias, "audio ffn_out");
}

}  // namespace

int32_t qwh_audio_layer(qwh_ctx *ctx, const qwh_audio_layer_weights *w, float *encoder_dev, uint32_t steps,
                        uint32_t d_model, uint32_t heads, uint32_t ffn_dim, uint32_t window_steps, float eps) {
    if (!ctx || !w) return QWH_E_INVALID_ARGUMENT;
    if (steps == 0) return QWH_OK;
    if (heads == 0 || d_model % heads != 0)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "d_model %u is not a multiple of %u heads", d_model, heads);
    if (window_steps == 0) return fail(ctx, QWH_E_INVALID_ARGUMENT, "window_steps is 0");
    QWH_TRY(check_device_ptr(ctx, encoder_dev, "encoder"));
    QWH_TRY(check_audio_matrix(ctx, w->q, d_model, d_model, "q"));
    QWH_TRY(check_audio_matrix(ctx, w->k, d_model, d_model, "k"));
    QWH_TRY(check_audio_matrix(ctx, w->v, d_model, d_model, "v"));
    QWH_TRY(check_audio_matrix(ctx, w->o, d_model, d_model, "o"));
    QWH_TRY(check_audio_matrix(ctx, w->ffn_in, ffn_dim, d_model, "ffn_in"));
    QWH_TRY(check_audio_matrix(ctx, w->ffn_out, d_model, ffn_dim, "ffn_out"));
    const void *vectors[] = {w->q_bias, w->k_bias, w->v_bias, w->o_bias, w->ffn_in_bias, w->ffn_out_bias,
                             w->attention_norm_weight, w->attention_norm_bias, w->final_norm_weight,
                             w->final_norm_bias};
    for (const void *p : vectors) QWH_TRY(check_device_ptr(ctx, p, "layer vector"));
    // Every check before the first launch, so a refused call leaves the
    // residual stream untouched: the linears' token limit (the batch GEMV's
    // grid rows), the attention's shape, and the 16-byte loads of ffn_in's
    // bias by ffn_out's activation prep.
    if (steps > 65535) return fail(ctx, QWH_E_LIMIT_EXCEEDED, "steps %u > 65535", steps);
    if (((uintptr_t)w->ffn_in_bias & 15u) != 0 || ((uintptr_t)encoder_dev & 15u) != 0)
        return fail(ctx, QWH_E_INVALID_ARGUMENT, "encoder and ffn_in bias must be 16-byte aligned");
    if (d_model % 4u || ffn_dim % 64u)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "d_model %u / ffn_dim %u: whole float4 rows and groups of 64", d_model,
                    ffn_dim);
    const size_t plane = (size_t)steps * d_model;
    QWH_TRY(ensure_workspace(ctx, ctx->audio, sizeof(float) * (5 * plane + (size_t)steps * ffn_dim)));
    float *normed = static_cast<float *>(ctx->audio.ptr);
    float *q = normed + plane, *k = q + plane, *v = k + plane, *block = v + plane, *wide = block + plane;
    hipStream_t s = ctx->stream;
    // :792-822 runWindowedAttention's arguments.
    AudioAttentionArgs a;
    a.out = block, a.q = q, a.k = k, a.v = v;
    a.q_bias = w->q_bias, a.k_bias = w->k_bias, a.v_bias = w->v_bias;
    a.out_stride = a.q_stride = a.k_stride = a.v_stride = d_model;
    a.first = 0, a.end = steps, a.window_steps = window_steps;
    a.heads = heads, a.head_dim = d_model / heads;
    a.scaling = 1.0f / sqrtf((float)a.head_dim);
    QWH_TRY(check_audio_attention(ctx, a));

    if (steps >= 2 && d_model % 64 == 0 && batch_ready(ctx, {w->q, w->k, w->v, w->o, w->ffn_in}, d_model) &&
        batch_ready(ctx, {w->ffn_out}, ffn_dim))
        return audio_layer_batch(ctx, w, encoder_dev, steps, d_model, ffn_dim, eps, a, wide);

    // model.zig:657-665 layerNormInto, :765-786 projectQkv (biases join in the attention's loads).
    QWH_TRY(check_hip(ctx, launch_layer_norm(s, encoder_dev, normed, w->attention_norm_weight, w->attention_norm_bias,
                                             d_model, steps, eps), "audio attention norm"));
    QWH_TRY(linear_shared_input(ctx, {w->q, w->k, w->v}, normed, d_model, steps, {q, k, v}));
    QWH_TRY(check_hip(ctx, launch_audio_attention(s, a), "audio attention"));
    // :824-848 projectAttentionOutput, :669 addInPlace.
    QWH_TRY(qwh_linear(ctx, w->o, block, d_model, steps, normed));
    QWH_TRY(check_hip(ctx, launch_bias_epilogue(s, kBiasResidual, normed, w->o_bias, encoder_dev, d_model, steps),
                      "audio o bias + residual"));
    // :671-679 layerNormInto, :852-872 activateFfn, :692 addInPlace.
    QWH_TRY(check_hip(ctx, launch_layer_norm(s, encoder_dev, normed, w->final_norm_weight, w->final_norm_bias, d_model,
                                             steps, eps), "audio final norm"));
    QWH_TRY(qwh_linear(ctx, w->ffn_in, normed, d_model, steps, wide));
    const Matrix *ffn_out = find_matrix(ctx, w->ffn_out);
    if (gemv_batch_supported(*ffn_out) && ((uintptr_t)ffn_out->data & 15u) == 0 && steps >= 2) {
        // The bias and GELU are applied as ffn_out's activation prep reads
        // `wide` (one pass and one launch fewer than a separate epilogue).
        const size_t parts = batch_partial_bytes(steps, *ffn_out);
        QWH_TRY(ensure_workspace(ctx, ctx->digits, batch_digit_bytes(steps, ffn_dim)));
        if (parts) QWH_TRY(ensure_workspace(ctx, ctx->scratch, parts));
        GemvInput in;
        in.mode = GemvInput::F32;
        in.x = wide;
        in.gelu_bias = w->ffn_in_bias;
        QWH_TRY(check_hip(ctx, launch_prep_batch(s, in, steps, ffn_dim, ctx->digits.ptr), "audio ffn prep"));
        QWH_TRY(check_hip(ctx, launch_gemv_batch(s, ctx->digits.ptr, *ffn_out, steps, block, nullptr, false,
                                                    static_cast<float *>(ctx->scratch.ptr)),
                          "audio ffn_out"));
    } else {
        QWH_TRY(check_hip(ctx, launch_bias_epilogue(s, kBiasGelu, wide, w->ffn_in_bias, nullptr, ffn_dim, steps),
                          "audio ffn bias + gelu"));
        QWH_TRY(qwh_linear(ctx, w->ffn_out, wide, ffn_dim, steps, block));
    }
    return check_hip(ctx, launch_bias_epilogue(s, kBiasResidual, block, w->ffn_out_bias, encoder_dev, d_model, steps),
                     "audio ffn bias + residual");
}

int32_t qwh_conv3x3s2_gelu(qwh_ctx *ctx, float *out_dev, const float *in_dev, const uint16_t *weights_dev,
                           const float *bias_dev, uint32_t batch, uint32_t out_channels, uint32_t in_channels,
                           uint32_t in_height, uint32_t in_width) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    // kernels.zig:344-349: a kernel of 3, non-empty planes and channels.
    if (in_height == 0 || in_width == 0 || in_channels == 0 || out_channels == 0)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "empty convolution geometry");
    if (batch == 0) return QWH_OK;
    const uint32_t oh = (in_height - 1) / 2 + 1, ow = (in_width - 1) / 2 + 1;
    if ((uint64_t)((oh + 7) / 8) * ((ow + 7) / 8) > 0xFFFFFFFFull || batch > 65535)
        return fail(ctx, QWH_E_LIMIT_EXCEEDED, "%u images of %u x %u", batch, in_height, in_width);
    QWH_TRY(check_device_ptr(ctx, out_dev, "out"));
    QWH_TRY(check_device_ptr(ctx, in_dev, "input"));
    QWH_TRY(check_device_ptr(ctx, weights_dev, "weights"));
    QWH_TRY(check_device_ptr(ctx, bias_dev, "bias"));
    if (conv_mfma_supported(in_channels, in_height, in_width)) {
        // The matrix-core form: the weights prepared into the context's
        // scratch, then the convolution.
        QWH_TRY(ensure_workspace(ctx, ctx->scratch, conv_mfma_prep_bytes(out_channels, in_channels)));
        QWH_TRY(check_hip(ctx, launch_conv_mfma_prep(ctx->stream, weights_dev, out_channels, in_channels,
                                                     ctx->scratch.ptr), "conv weight prep"));
        return check_hip(ctx, launch_conv3x3s2_gelu_mfma(ctx->stream, out_dev, in_dev, ctx->scratch.ptr, bias_dev, batch,
                                                         out_channels, in_channels, in_height, in_width),
                         "conv3x3 stride 2");
    }
    return check_hip(ctx, launch_conv3x3s2_gelu(ctx->stream, out_dev, in_dev, weights_dev, bias_dev, batch, out_channels,
                                                in_channels, in_height, in_width), "conv3x3 stride 2");
}

namespace {

// model_config.zig:84-90 postConvolutionSteps: three (n - 1) / 2 + 1.
uint32_t post_convolution(uint32_t n) {
    if (n == 0) return 0;
    for (int i = 0; i < 3; ++i) n = (n - 1) / 2 + 1;
    return n;
}

}  // namespace

int32_t qwh_audio_frontend(qwh_ctx *ctx, const qwh_audio_frontend_weights *w, const float *log_mel_dev,
                           uint32_t mel_bins, uint32_t frames, uint32_t n_window, uint32_t downsample,
                           uint32_t d_model, float *encoder_dev, uint32_t encoder_rows, uint32_t *steps_out) {
    if (!ctx || !w || !steps_out) return QWH_E_INVALID_ARGUMENT;
    *steps_out = 0;
    if (mel_bins == 0 || n_window == 0 || downsample == 0 || d_model == 0 || d_model % 2)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "mel_bins, n_window, downsample and an even d_model are required");
    const uint32_t chunk_frames = 2 * n_window;       // model_config.zig:196-198
    const uint32_t chunk_steps = post_convolution(chunk_frames);
    const uint32_t bins = post_convolution(mel_bins);  // audioFrequencyBinsAfterConvolutions
    const uint32_t features = downsample * bins;       // audioConvOutInputFeatures
    const Matrix *proj = find_matrix(ctx, w->conv_out);
    if (!proj) return fail(ctx, QWH_E_NOT_FOUND, "unknown conv_out matrix handle");
    if (proj->rows != d_model || proj->cols != features)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "conv_out is %u x %u, the front end needs %u x %u", proj->rows,
                    proj->cols, d_model, features);
    // model_config.zig:226-238 audio steps of the clip.
    const uint32_t chunks = (frames + chunk_frames - 1) / chunk_frames;
    const uint64_t steps = (uint64_t)(frames / chunk_frames) * chunk_steps + post_convolution(frames % chunk_frames);
    if (steps > encoder_rows)
        return fail(ctx, QWH_E_LIMIT_EXCEEDED, "%llu encoder rows needed, %u given", (unsigned long long)steps,
                    encoder_rows);
    if (steps == 0) return QWH_OK;
    QWH_TRY(check_device_ptr(ctx, log_mel_dev, "log_mel"));
    QWH_TRY(check_device_ptr(ctx, encoder_dev, "encoder"));
    const void *vectors[] = {w->conv1_weight, w->conv2_weight, w->conv3_weight, w->conv1_bias, w->conv2_bias,
                             w->conv3_bias};
    for (const void *p : vectors) QWH_TRY(check_device_ptr(ctx, p, "front-end weight"));
    if (((uintptr_t)encoder_dev & 15u) != 0) return fail(ctx, QWH_E_INVALID_ARGUMENT, "encoder must be 16-byte aligned");
    // The three stages' planes per chunk, in chunk groups of at most 32.
    const uint32_t h1 = (mel_bins - 1) / 2 + 1, w1 = (chunk_frames - 1) / 2 + 1;
    const uint32_t h2 = (h1 - 1) / 2 + 1, w2 = (w1 - 1) / 2 + 1;
    const size_t mel_plane = (size_t)mel_bins * chunk_frames;
    const size_t p1 = (size_t)downsample * h1 * w1, p2 = (size_t)downsample * h2 * w2;
    const size_t p3 = (size_t)downsample * bins * chunk_steps;
    const uint32_t group = chunks < 32 ? chunks : 32;
    auto align = [](size_t n) { return (n + 63) & ~(size_t)63; };  // floats: 256-byte aligned pieces
    const size_t off1 = align(group * mel_plane), off2 = off1 + align(group * p1), off3 = off2 + align(group * p2);
    const size_t off_flat = off3 + align(group * p3);
    // conv2 / conv3 on the matrix cores where their shapes allow: their
    // weights prepared once per call after the planes.
    const bool mfma2 = conv_mfma_supported(downsample, h1, w1), mfma3 = conv_mfma_supported(downsample, h2, w2);
    const size_t prep_floats = align(conv_mfma_prep_bytes(downsample, downsample) / sizeof(float));
    const size_t off_prep2 = off_flat + align((size_t)group * chunk_steps * features);
    const size_t off_prep3 = off_prep2 + (mfma2 ? prep_floats : 0);
    const size_t total = off_prep3 + (mfma3 ? prep_floats : 0);
    QWH_TRY(ensure_workspace(ctx, ctx->front, total * sizeof(float)));
    float *ws = static_cast<float *>(ctx->front.ptr);
    hipStream_t s = ctx->stream;
    if (mfma2)
        QWH_TRY(check_hip(ctx, launch_conv_mfma_prep(s, w->conv2_weight, downsample, downsample, ws + off_prep2),
                          "conv2 weight prep"));
    if (mfma3)
        QWH_TRY(check_hip(ctx, launch_conv_mfma_prep(s, w->conv3_weight, downsample, downsample, ws + off_prep3),
                          "conv3 weight prep"));
    if (!ctx->front_table.ptr || ctx->front_table_steps != chunk_steps || ctx->front_table_width != d_model) {
        // addSinusoidalPosition (model.zig:751-763) for the steps of a chunk,
        // in f64 on the host, narrowed to f32 as the reference does; built
        // once per shape and kept on the device.
        std::vector<float> table((size_t)chunk_steps * d_model, 0.0f);
        const uint32_t half = d_model / 2;
        const double increment = std::log(10000.0) / ((double)half - 1.0);
        for (uint32_t step = 0; step < chunk_steps; ++step)
            for (uint32_t i = 0; i < half; ++i) {
                const double angle = (double)step * std::exp(-increment * (double)i);
                table[(size_t)step * d_model + i] = (float)std::sin(angle);
                table[(size_t)step * d_model + half + i] = (float)std::cos(angle);
            }
        ctx->front_table_steps = 0;
        QWH_TRY(ensure_workspace(ctx, ctx->front_table, table.size() * sizeof(float)));
        QWH_TRY(check_hip(ctx, hipMemcpyAsync(ctx->front_table.ptr, table.data(), table.size() * 4,
                                              hipMemcpyHostToDevice, s), "position table"));
        // The copy reads host memory owned by this call.
        QWH_TRY(check_hip(ctx, hipStreamSynchronize(s), "position table"));
        ctx->front_table_steps = chunk_steps;
        ctx->front_table_width = d_model;
    }
    const float *pos_table = static_cast<const float *>(ctx->front_table.ptr);
    for (uint32_t c0 = 0; c0 < chunks; c0 += group) {
        const uint32_t count = chunks - c0 < group ? chunks - c0 : group;
        const uint32_t row0 = c0 * chunk_steps;  // every chunk before the last is whole
        const uint32_t rows = (uint32_t)(steps - row0 < (uint64_t)count * chunk_steps ? steps - row0 : count * chunk_steps);
        QWH_TRY(check_hip(ctx, launch_gather_chunks(s, log_mel_dev, mel_bins, frames, chunk_frames, c0, count, ws),
                          "front-end chunks"));
        QWH_TRY(check_hip(ctx, launch_conv3x3s2_gelu(s, ws + off1, ws, w->conv1_weight, w->conv1_bias, count, downsample,
                                                     1, mel_bins, chunk_frames), "conv1"));
        QWH_TRY(check_hip(ctx, mfma2 ? launch_conv3x3s2_gelu_mfma(s, ws + off2, ws + off1, ws + off_prep2,
                                                                  w->conv2_bias, count, downsample, downsample, h1, w1)
                                     : launch_conv3x3s2_gelu(s, ws + off2, ws + off1, w->conv2_weight, w->conv2_bias,
                                                             count, downsample, downsample, h1, w1),
                          "conv2"));
        QWH_TRY(check_hip(ctx, mfma3 ? launch_conv3x3s2_gelu_mfma(s, ws + off3, ws + off2, ws + off_prep3,
                                                                  w->conv3_bias, count, downsample, downsample, h2, w2)
                                     : launch_conv3x3s2_gelu(s, ws + off3, ws + off2, w->conv3_weight, w->conv3_bias,
                                                             count, downsample, downsample, h2, w2),
                          "conv3"));
        QWH_TRY(check_hip(ctx, launch_pack_steps(s, ws + off3, downsample, bins, chunk_steps, rows, ws + off_flat),
                          "front-end flatten"));
        float *out = encoder_dev + (size_t)row0 * d_model;
        QWH_TRY(qwh_linear(ctx, w->conv_out, ws + off_flat, features, rows, out));
        QWH_TRY(check_hip(ctx, launch_add_positions(s, out, pos_table, row0, rows, d_model, chunk_steps),
                          "front-end positions"));
    }
    *steps_out = (uint32_t)steps;
    return QWH_OK;
}

int32_t qwh_argmax_rows(qwh_ctx *ctx, const float *logits_dev, uint32_t rows, uint32_t count, uint32_t *ids_dev) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    if (rows == 0) return QWH_OK;
    if (count == 0) return fail(ctx, QWH_E_INVALID_ARGUMENT, "argmax over an empty row");
    if (rows > 65535) return fail(ctx, QWH_E_LIMIT_EXCEEDED, "rows %u > 65535", rows);
    QWH_TRY(check_device_ptr(ctx, logits_dev, "logits"));
    QWH_TRY(check_device_ptr(ctx, ids_dev, "ids"));
    QWH_TRY(ensure_workspace(ctx, ctx->scratch, argmax_scratch_bytes(rows, count)));
    return check_hip(ctx, launch_argmax_rows(ctx->stream, logits_dev, rows, count, ctx->scratch.ptr, ids_dev),
                     "argmax");
}

int32_t qwh_audio_projector(qwh_ctx *ctx, uint64_t in_matrix, const float *in_bias_dev, uint64_t out_matrix,
                            const float *out_bias_dev, const float *encoder_dev, uint32_t steps, float *out_dev) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    const Matrix *mi = find_matrix(ctx, in_matrix);
    const Matrix *mo = find_matrix(ctx, out_matrix);
    if (!mi || !mo) return fail(ctx, QWH_E_NOT_FOUND, "unknown projector matrix handle");
    // model.zig:707-735: in is d_model x d_model, out is hidden x d_model.
    if (mi->rows != mi->cols || mo->cols != mi->rows)
        return fail(ctx, QWH_E_SHAPE_MISMATCH, "projector matrices %u x %u and %u x %u do not chain", mi->rows, mi->cols,
                    mo->rows, mo->cols);
    if (steps == 0) return QWH_OK;
    QWH_TRY(check_device_ptr(ctx, in_bias_dev, "in bias"));
    QWH_TRY(check_device_ptr(ctx, out_bias_dev, "out bias"));
    QWH_TRY(check_device_ptr(ctx, out_dev, "out"));
    QWH_TRY(ensure_workspace(ctx, ctx->audio, sizeof(float) * (size_t)steps * mi->rows));
    float *mid = static_cast<float *>(ctx->audio.ptr);
    const uint32_t d_model = mi->rows, hidden = mo->rows;
    QWH_TRY(qwh_linear(ctx, in_matrix, encoder_dev, d_model, steps, mid));
    QWH_TRY(check_hip(ctx, launch_bias_epilogue(ctx->stream, kBiasGelu, mid, in_bias_dev, nullptr, d_model, steps),
                      "projector bias + gelu"));
    QWH_TRY(qwh_linear(ctx, out_matrix, mid, d_model, steps, out_dev));
    return check_hip(ctx, launch_bias_epilogue(ctx->stream, kBiasAdd, out_dev, out_bias_dev, nullptr, hidden, steps),
                     "projector bias");
}

}  // extern "C"
