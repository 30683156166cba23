// CPU check of the decode attention's scratch sizing (attention_plan.h),
// built with g++ only: for every shape and form the decoder step, the
// prefill and the attention entry points launch, the bytes they allocate
// (sized before the launch form is known) hold the records of the ranges
// the launch then writes. Exit status 0 when every case holds.
#include <cstdio>

#include "../csrc/attention_plan.h"

using qwh::AttentionArgs;
namespace plan = qwh::plan;

namespace {

struct Heads {
    uint32_t heads, kv_heads, head_dim;
};

long cases = 0, failures = 0;

// `sized`: the bytes the caller allocated; the launch writes the records of
// the form it takes (decoder: q / k norms given).
void check(const char *who, int cus, const AttentionArgs &a, bool decoder, size_t sized) {
    uint32_t chunk = 0, splits = 0;
    plan::attention_shape(cus, a, decoder, chunk, splits);
    const size_t need = plan::record_bytes(a, splits);
    ++cases;
    // Every range starts below the capacity and the ranges cover it.
    const bool ranges_ok = splits >= 1 && (uint64_t)(splits - 1) * chunk < a.capacity &&
                           (uint64_t)splits * chunk >= a.capacity && chunk % (plan::kTile * plan::kWaves) == 0;
    if (need > sized || !ranges_ok) {
        ++failures;
        if (failures <= 20)
            std::printf("FAIL %s: cus %d heads %u/%u d %u batch %u capacity %u f32 %d decoder %d: "
                        "splits %u chunk %u need %zu sized %zu\n",
                        who, cus, a.heads, a.kv_heads, a.head_dim, a.batch, a.capacity, (int)a.f32_cache,
                        (int)decoder, splits, chunk, need, sized);
    }
}

}  // namespace

int main() {
    // The Qwen3-ASR decoders (0.6B: 16 / 8 heads of 128; 1.7B the same
    // heads), the test suites' shapes, and every head layout the kernels
    // are built for.
    const Heads heads[] = {{16, 8, 128}, {4, 2, 128}, {5, 5, 64}, {8, 2, 64}, {16, 2, 128}, {16, 4, 64},
                           {2, 2, 256}, {4, 2, 256}, {8, 8, 128}, {64, 8, 128}};
    const int cus_list[] = {256, 304, 80, 1};
    const uint32_t capacities[] = {1, 2, 31, 64, 127, 128, 255, 256, 257, 600, 4096, 4352, 8192};
    for (const Heads &h : heads)
        for (int cus : cus_list)
            for (uint32_t capacity : capacities)
                for (uint32_t batch = 1; batch <= 300; batch += batch < 20 ? 1 : 37)
                    for (int f32 = 0; f32 < 2; ++f32) {
                        AttentionArgs a{};
                        a.heads = h.heads;
                        a.kv_heads = h.kv_heads;
                        a.head_dim = h.head_dim;
                        a.batch = batch;
                        a.capacity = capacity;
                        a.f32_cache = f32 != 0;
                        // The decoder sizes its scratch at create, before the
                        // norm pointers exist, and launches the decoder form.
                        const size_t at_create = plan::scratch_bytes(cus, a);
                        check("decoder step", cus, a, true, at_create);
                        // The attention entry points size and launch the
                        // plain form.
                        check("entry point", cus, a, false, at_create);
                        // The prefill sizes with its chunk's rows as the batch
                        // and the positions through the chunk as the capacity,
                        // norm pointers given, and launches the decoder form.
                        AttentionArgs p = a;
                        p.prefill = true;
                        check("prefill", cus, p, true, plan::scratch_bytes(cus, p));
                    }
    std::printf("attention scratch sizing: %ld cases, %ld failures\n", cases, failures);
    return failures ? 1 : 0;
}
