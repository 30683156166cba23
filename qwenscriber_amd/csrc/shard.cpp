// `.qw` weight shards (container.zig) into device memory.
//
// A shard is a 32-byte header, an index of 40-byte entries sorted by
// (layer, kind), and a payload that starts on a 256-byte boundary and holds
// every tensor at a 16-byte aligned offset (quantized tensors as the two
// quant.planeLayout planes). Validation follows container.zig File.parse
// rule by rule and in the same order, so a shard is rejected with the status
// the reference's ABI maps the same error to (wasm/abi.zig:90-146). It runs
// on the host and needs no device: qwh_shard_validate / _find /
// _verify_checksum take the file bytes.
//
// qwh_shard_load validates a shard and copies its payload to the device in
// one piece; tensors are then addressed inside that allocation without
// further copies: qwh_shard_matrix hands out a matrix handle that borrows a
// quantized tensor's planes (as qwh_matrix_wrap does), qwh_shard_tensor the
// device address of any tensor. A shard cannot be released while a matrix
// still borrows from it.
#include <cstring>

#include "common.h"

namespace qwh {
namespace {

constexpr uint32_t kHeaderBytes = 32;     // container.zig:60
constexpr uint32_t kEntryBytes = 40;      // container.zig:61
constexpr uint64_t kPayloadAlign = 256;   // container.zig:64
constexpr uint64_t kTensorAlign = 16;     // quant.tensor_alignment_bytes
constexpr uint32_t kMaxDim = 1u << 24;    // tensor.zig:21 dims_max
const char kMagic[8] = {'Q', 'W', 'S', 'H', 'A', 'R', 'D', '1'};

uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }

struct Header {
    uint32_t version, index_len, payload_offset, payload_len, count, checksum;
};

uint64_t align_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

bool known_format(uint8_t f) { return f == 0 || f == 1 || f == 2 || f == QWH_FORMAT_Q4 || f == QWH_FORMAT_Q5 || f == QWH_FORMAT_Q8; }
bool quantized(uint8_t f) { return f == QWH_FORMAT_Q4 || f == QWH_FORMAT_Q5 || f == QWH_FORMAT_Q8; }
uint32_t element_bytes(uint8_t f) { return f == 0 ? 4 : 2; }

// quant.planeLayout (quant.zig:144-176) of a rows x cols matrix placed at
// `base`: the scale plane at the first 16-byte boundary, the data plane at
// the next one after it. Offsets are relative to `base`.
struct Planes {
    uint64_t scales_off, scales_len, data_off, data_len, total;
};
bool plane_layout(uint8_t format, uint32_t rows, uint32_t cols, uint64_t base, Planes &p) {
    if (cols % 64 != 0) return false;
    const uint64_t groups = (uint64_t)rows * (cols / 64);
    p.scales_len = groups * 2;
    p.data_len = groups * (format == QWH_FORMAT_Q4 ? 32u : format == QWH_FORMAT_Q5 ? 40u : 64u);
    p.scales_off = align_up(base, kTensorAlign) - base;
    p.data_off = align_up(base + p.scales_off + p.scales_len, kTensorAlign) - base;
    p.total = p.data_off + p.data_len;
    return true;
}

// Entry.validate (container.zig:142-160): a known format, a shape the format
// accepts, and a recorded length equal to the one the shape implies.
int32_t validate_entry(const qwh_tensor_entry &e) {
    if (!known_format(e.format)) return QWH_E_UNSUPPORTED_MODEL;  // UnsupportedFormat
    // tensor.Shape.fromDims: rank 1..4, every extent in 1..2^24.
    if (e.rank == 0 || e.rank > 4) return QWH_E_SHAPE_MISMATCH;
    for (int i = 0; i < e.rank; ++i)
        if (e.dims[i] == 0 || e.dims[i] > kMaxDim) return QWH_E_SHAPE_MISMATCH;
    uint64_t expected;
    if (quantized(e.format)) {
        // Shape.validateForFormat: a matrix whose rows are whole groups.
        if (e.rank != 2 || e.dims[1] % 64 != 0) return QWH_E_SHAPE_MISMATCH;
        Planes p;
        plane_layout(e.format, e.dims[0], e.dims[1], 0, p);
        expected = p.total;
    } else {
        // Shape.elementCount and the byte count, overflow checked
        // (CountOverflow maps to ShapeMismatch here).
        uint64_t count = 1;
        for (int i = 0; i < e.rank; ++i)
            if (__builtin_mul_overflow(count, (uint64_t)e.dims[i], &count)) return QWH_E_SHAPE_MISMATCH;
        if (__builtin_mul_overflow(count, (uint64_t)element_bytes(e.format), &expected)) return QWH_E_SHAPE_MISMATCH;
    }
    if (expected != e.len_bytes) return QWH_E_SHAPE_MISMATCH;  // ByteLengthMismatch
    if (quantized(e.format)) {
        Planes p;
        plane_layout(e.format, e.dims[0], e.dims[1], e.offset_bytes, p);
        if (p.total != e.len_bytes || p.scales_off != 0) return QWH_E_SHAPE_MISMATCH;  // ByteLengthMismatch
    }
    return QWH_OK;
}

qwh_tensor_entry read_entry(const uint8_t *p) {
    qwh_tensor_entry e{};
    e.kind = rd16(p);
    e.layer = rd16(p + 2);
    e.format = p[4];
    e.rank = p[5];
    e.reserved = rd16(p + 6);
    for (int i = 0; i < 4; ++i) e.dims[i] = rd32(p + 8 + 4 * i);
    e.offset_bytes = rd64(p + 24);
    e.len_bytes = rd64(p + 32);
    return e;
}

uint32_t sort_key(uint16_t layer, uint16_t kind) { return ((uint32_t)layer << 16) | kind; }

// File.parse + File.validate (container.zig:175-217). On success `h` holds
// the header and `index` points at the first entry.
int32_t parse(const void *bytes, uint64_t len, Header &h, const uint8_t *&index) {
    if (!bytes) return QWH_E_INVALID_ARGUMENT;
    const uint8_t *b = static_cast<const uint8_t *>(bytes);
    if (len < kHeaderBytes) return QWH_E_TRUNCATED;
    // Header.validate (container.zig:88-99).
    if (std::memcmp(b, kMagic, 8) != 0) return QWH_E_BAD_MAGIC;
    h.version = rd32(b + 8);
    h.index_len = rd32(b + 12);
    h.payload_offset = rd32(b + 16);
    h.payload_len = rd32(b + 20);
    h.count = rd32(b + 24);
    h.checksum = rd32(b + 28);
    if (h.version != 1) return QWH_E_BAD_VERSION;
    if ((uint64_t)h.index_len != (uint64_t)h.count * kEntryBytes) return QWH_E_TRUNCATED;
    if ((uint64_t)h.payload_offset < (uint64_t)kHeaderBytes + h.index_len) return QWH_E_TRUNCATED;
    if (h.payload_offset % kPayloadAlign != 0) return QWH_E_TRUNCATED;
    if (len < (uint64_t)kHeaderBytes + h.index_len) return QWH_E_TRUNCATED;
    if (len < (uint64_t)h.payload_offset + h.payload_len) return QWH_E_TRUNCATED;
    index = b + kHeaderBytes;
    uint64_t previous_end = 0;
    uint32_t previous_key = 0;
    for (uint32_t i = 0; i < h.count; ++i) {
        const qwh_tensor_entry e = read_entry(index + (size_t)i * kEntryBytes);
        const int32_t st = validate_entry(e);
        if (st != QWH_OK) return st;
        const uint32_t key = sort_key(e.layer, e.kind);
        if (i > 0 && key <= previous_key) return QWH_E_INVALID_ARGUMENT;  // IndexNotSorted
        previous_key = key;
        if (e.offset_bytes < previous_end) return QWH_E_INVALID_ARGUMENT;  // TensorRangesOverlap
        const uint64_t end = e.offset_bytes + e.len_bytes;
        if (end < e.offset_bytes || end > h.payload_len) return QWH_E_TRUNCATED;
        previous_end = end;
        if (e.offset_bytes % kTensorAlign != 0) return QWH_E_INVALID_ARGUMENT;  // TensorRangesOverlap
    }
    return QWH_OK;
}

// File.find (container.zig:226-236): the index is sorted, so the scan stops
// once the key is passed.
bool find_entry(const uint8_t *index, uint32_t count, uint16_t kind, uint16_t layer, qwh_tensor_entry &out) {
    const uint32_t key = sort_key(layer, kind);
    for (uint32_t i = 0; i < count; ++i) {
        const qwh_tensor_entry e = read_entry(index + (size_t)i * kEntryBytes);
        const uint32_t k = sort_key(e.layer, e.kind);
        if (k == key) {
            out = e;
            return true;
        }
        if (k > key) return false;
    }
    return false;
}

// Low 32 bits of FNV-1a 64 over the payload (container.zig:279-281).
uint32_t payload_checksum(const uint8_t *p, uint64_t n) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (uint64_t i = 0; i < n; ++i) {
        h ^= p[i];
        h *= 0x100000001b3ull;
    }
    return (uint32_t)h;
}

}  // namespace
}  // namespace qwh

using namespace qwh;

extern "C" {

int32_t qwh_shard_validate(const void *bytes, uint64_t len, uint32_t *tensor_count) {
    Header h;
    const uint8_t *index;
    const int32_t st = parse(bytes, len, h, index);
    if (st == QWH_OK && tensor_count) *tensor_count = h.count;
    return st;
}

int32_t qwh_shard_verify_checksum(const void *bytes, uint64_t len) {
    Header h;
    const uint8_t *index;
    const int32_t st = parse(bytes, len, h, index);
    if (st != QWH_OK) return st;
    const uint8_t *payload = static_cast<const uint8_t *>(bytes) + h.payload_offset;
    return payload_checksum(payload, h.payload_len) == h.checksum ? QWH_OK : QWH_E_CHECKSUM_MISMATCH;
}

int32_t qwh_shard_find(const void *bytes, uint64_t len, uint16_t kind, uint16_t layer, qwh_tensor_entry *out) {
    if (!out) return QWH_E_INVALID_ARGUMENT;
    Header h;
    const uint8_t *index;
    const int32_t st = parse(bytes, len, h, index);
    if (st != QWH_OK) return st;
    return find_entry(index, h.count, kind, layer, *out) ? QWH_OK : QWH_E_NOT_FOUND;
}

int32_t qwh_shard_load(qwh_ctx *ctx, const void *bytes, uint64_t len, uint64_t *out_shard) {
    if (!ctx || !out_shard) return QWH_E_INVALID_ARGUMENT;
    Header h;
    const uint8_t *index;
    const int32_t st = parse(bytes, len, h, index);
    if (st != QWH_OK) return fail(ctx, st, "shard rejected (container.zig File.parse)");
    Shard s;
    s.payload_len = h.payload_len;
    s.index.resize(h.count);
    for (uint32_t i = 0; i < h.count; ++i) s.index[i] = read_entry(index + (size_t)i * 40u);
    const size_t bytes_dev = (size_t)align_up(h.payload_len ? h.payload_len : 1, kPayloadAlign);
    QWH_TRY(check_hip(ctx, hipMalloc(&s.payload, bytes_dev), "shard payload alloc"));
    const uint8_t *payload = static_cast<const uint8_t *>(bytes) + h.payload_offset;
    const int32_t up = check_hip(ctx, hipMemcpyAsync(s.payload, payload, h.payload_len, hipMemcpyHostToDevice,
                                                     ctx->stream), "shard payload upload");
    if (up == QWH_OK) {
        const int32_t sync = check_hip(ctx, hipStreamSynchronize(ctx->stream), "shard payload upload");
        if (sync != QWH_OK) {
            (void)hipFree(s.payload);
            return sync;
        }
    } else {
        (void)hipFree(s.payload);
        return up;
    }
    const uint64_t handle = ctx->next_handle++;
    ctx->shards[handle] = std::move(s);
    *out_shard = handle;
    return QWH_OK;
}

int32_t qwh_shard_tensor(qwh_ctx *ctx, uint64_t shard, uint16_t kind, uint16_t layer, void **dev,
                         qwh_tensor_entry *entry) {
    if (!ctx || !dev) return QWH_E_INVALID_ARGUMENT;
    auto it = ctx->shards.find(shard);
    if (it == ctx->shards.end()) return fail(ctx, QWH_E_NOT_FOUND, "unknown shard handle %llu", (unsigned long long)shard);
    const Shard &s = it->second;
    const uint32_t key = ((uint32_t)layer << 16) | kind;
    for (const qwh_tensor_entry &e : s.index) {
        const uint32_t k = ((uint32_t)e.layer << 16) | e.kind;
        if (k == key) {
            *dev = static_cast<uint8_t *>(s.payload) + e.offset_bytes;
            if (entry) *entry = e;
            return QWH_OK;
        }
        if (k > key) break;
    }
    return fail(ctx, QWH_E_NOT_FOUND, "no tensor kind %u layer %u in the shard", kind, layer);
}

int32_t qwh_shard_matrix(qwh_ctx *ctx, uint64_t shard, uint16_t kind, uint16_t layer, uint64_t *out_matrix) {
    if (!ctx || !out_matrix) return QWH_E_INVALID_ARGUMENT;
    void *dev = nullptr;
    qwh_tensor_entry e{};
    QWH_TRY(qwh_shard_tensor(ctx, shard, kind, layer, &dev, &e));
    if (is_dense_format(e.format) && e.rank == 2) {
        // model.zig:92-96 Binding.matrix: an f32 / f16 tensor's elements, in
        // place, as a dims[0] x dims[1] matrix.
        Matrix m;
        m.format = e.format;
        m.rows = e.dims[0];
        m.cols = e.dims[1];
        m.data = static_cast<uint8_t *>(dev);
        m.owned = false;
        m.shard = shard;
        *out_matrix = add_matrix(ctx, m);
        return QWH_OK;
    }
    // File.quantizedPlanes (container.zig:248-266): none for other element
    // tensors (bf16, or vectors).
    if (!quantized(e.format)) return fail(ctx, QWH_E_NOT_FOUND, "tensor kind %u layer %u is not a matrix", kind, layer);
    Planes p;
    plane_layout(e.format, e.dims[0], e.dims[1], e.offset_bytes, p);
    Matrix m;
    m.format = e.format;
    m.rows = e.dims[0];
    m.cols = e.dims[1];
    m.scales = static_cast<uint8_t *>(dev) + p.scales_off;
    m.data = static_cast<uint8_t *>(dev) + p.data_off;
    m.owned = false;
    m.shard = shard;
    *out_matrix = add_matrix(ctx, m);
    return QWH_OK;
}

int32_t qwh_shard_release(qwh_ctx *ctx, uint64_t shard) {
    if (!ctx) return QWH_E_INVALID_ARGUMENT;
    auto it = ctx->shards.find(shard);
    if (it == ctx->shards.end()) return fail(ctx, QWH_E_NOT_FOUND, "unknown shard handle %llu", (unsigned long long)shard);
    for (const auto &kv : ctx->matrices)
        if (kv.second.shard == shard)
            return fail(ctx, QWH_E_INVALID_STATE, "matrix %llu still borrows from shard %llu",
                        (unsigned long long)kv.first, (unsigned long long)shard);
    QWH_TRY(check_hip(ctx, hipStreamSynchronize(ctx->stream), "shard release sync"));
    (void)hipFree(it->second.payload);
    ctx->shards.erase(it);
    return QWH_OK;
}

}  // extern "C"
