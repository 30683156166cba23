// The decode attention's range plan (host arithmetic, no device code): how
// many positions each range workgroup scores, how many ranges a launch has,
// and the bytes of range records they write. attention.hip launches by it;
// sanitize/plan_check.cpp checks the scratch sizing against it on the CPU.
#pragma once

#include <cstddef>
#include <cstdint>

#include "common.h"

namespace qwh {
namespace plan {

constexpr uint32_t kTile = 32;        // positions per wavefront per iteration
constexpr uint32_t kWaves = 4;        // wavefronts per range workgroup
constexpr uint32_t kMaxSplits = 512;  // ranges per (sequence, kv head) at most

// Workgroups of the range kernel resident per CU: three where the kernel is
// compiled for three wavefronts per SIMD (the q8 forms of at most two query
// heads per kv head at head_dim 64, and at 128 for the decoder form), else
// two. (With the values on the matrix cores the decoder form also fits four
// wavefronts per SIMD; four resident workgroups, with the ranges that many
// more need, ran batch 16 at 7008 tokens/s against 7290.)
inline uint32_t resident_groups(const AttentionArgs &a, bool decoder) {
    const uint32_t ratio = a.heads / a.kv_heads;
    return !a.f32_cache && ratio <= 2 && (a.head_dim == 64 || (a.head_dim == 128 && decoder)) ? 3 : 2;
}

// Ranges of `chunk` positions for the decoder form (q/k norms given: the
// decoder step) or the plain form. Positions per workgroup: a multiple of
// one workgroup iteration of the q8 kernel (kTile * kWaves = 128 positions;
// the f32 kernel's iteration divides it), at least two of them; as many
// workgroups as the device holds at once, at most kMaxSplits ranges. (At
// batch 1, 128-position ranges spend more on the per-range query prologue
// and the combine than their extra workgroups win back: 17 ranges of 256
// beat 34 of 128 at 4096 positions.)
inline void attention_shape(int cus, const AttentionArgs &a, bool decoder, uint32_t &chunk, uint32_t &splits) {
    const uint32_t step = kTile * kWaves;
    const uint32_t target = (uint32_t)(cus > 0 ? cus : 256) * resident_groups(a, decoder);
    const uint32_t pairs = a.batch * a.kv_heads;
    uint32_t want_splits = (target + pairs - 1) / pairs;
    if (want_splits < 1) want_splits = 1;
    if (want_splits > kMaxSplits) want_splits = kMaxSplits;
    const uint32_t per = (a.capacity + want_splits - 1) / want_splits;
    chunk = ((per + step - 1) / step) * step;
    if (chunk < 2 * step) chunk = 2 * step;
    splits = (a.capacity + chunk - 1) / chunk;
    if (splits < 1) splits = 1;
}

// Bytes of the records `splits` ranges write: per (sequence, kv head, range)
// R * head_dim partial sums and 4 R softmax values, R query heads per kv head.
inline size_t record_bytes(const AttentionArgs &a, uint32_t splits) {
    const uint32_t R = a.heads / a.kv_heads;
    return (size_t)a.batch * a.kv_heads * splits * (R * a.head_dim + 4 * R) * sizeof(float) + 256;
}

// Enough for either form's ranges, so a buffer sized before the norm
// pointers are known (the decoder's) holds the decoder form's records.
inline size_t scratch_bytes(int cus, const AttentionArgs &a) {
    uint32_t chunk, plain, decoder;
    attention_shape(cus, a, false, chunk, plain);
    attention_shape(cus, a, true, chunk, decoder);
    return record_bytes(a, plain > decoder ? plain : decoder);
}

}  // namespace plan
}  // namespace qwh
