// Roofline calibration: a plain streaming read of a buffer, the ceiling the
// GEMVs are compared with. Each wavefront reads contiguous 4 KB chunks
// (chunk c = wave + k * waves: 64 lanes x four 16-byte non-temporal loads,
// all in flight together -- the fastest of the read patterns measured on
// MI355X for buffers of 80-170 MB) and folds them into one word with XOR so
// that no load is dead; one word per workgroup is written. Not part of the
// reference: the bench reports it next to the HBM peak.
#include "common.h"

namespace qwh {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4 *src, uint64_t pieces, uint32_t *sink) {
    constexpr uint64_t kChunk = 64 * 4;  // 16-byte pieces per chunk
    const int lane = threadIdx.x & 63;
    const uint64_t wave = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint64_t waves = ((uint64_t)gridDim.x * blockDim.x) >> 6;
    const uint64_t chunks = pieces / kChunk;
    u32x4 acc = {0u, 0u, 0u, 0u};
    for (uint64_t c = wave; c < chunks; c += waves) {
        const u32x4 *p = src + c * kChunk + lane;
        const u32x4 a = __builtin_nontemporal_load(p);
        const u32x4 b = __builtin_nontemporal_load(p + 64);
        const u32x4 d = __builtin_nontemporal_load(p + 128);
        const u32x4 e = __builtin_nontemporal_load(p + 192);
        acc ^= a ^ b ^ d ^ e;
    }
    // The pieces past the last whole chunk.
    for (uint64_t i = chunks * kChunk + wave * 64 + lane; i < pieces; i += waves * 64)
        acc ^= __builtin_nontemporal_load(src + i);
    uint32_t v = acc.x ^ acc.y ^ acc.z ^ acc.w;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v ^= (uint32_t)__shfl_xor((int)v, m, 64);
    __shared__ uint32_t waves_word[4];
    if ((threadIdx.x & 63) == 0) waves_word[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) sink[blockIdx.x] = waves_word[0] ^ waves_word[1] ^ waves_word[2] ^ waves_word[3];
}

}  // namespace

hipError_t launch_stream_read(hipStream_t s, int cus, const void *src, uint64_t bytes, uint32_t blocks_per_cu,
                              uint32_t *sink) {
    const uint64_t pieces = bytes / 16;
    const uint32_t blocks = (uint32_t)(cus > 0 ? cus : 256) * (blocks_per_cu ? blocks_per_cu : 4);
    stream_read_kernel<<<blocks, 256, 0, s>>>(static_cast<const u32x4 *>(src), pieces, sink);
    return hipGetLastError();
}

}  // namespace qwh
