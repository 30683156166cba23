// Host-only check of the untrusted-byte parsers under AddressSanitizer and
// UndefinedBehaviorSanitizer: container.File.parse / find / verifyChecksum
// (shard.cpp) and model_config.parse (config.cpp), over the files named on
// the command line and deterministic mutations of each (byte flips, 32- and
// 64-bit fields set to extreme values, truncations, appended bytes). Every
// input is copied into a heap buffer of exactly its length, so a read past
// the end is an ASan report. The statuses are not checked here (the Python
// tests do that); a sanitizer report aborts with a nonzero exit.
//
// Usage: parsers <mutations per file> <file>...
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "../../include/qwhip.h"

namespace {

uint64_t g_state = 0x9e3779b97f4a7c15ull;

uint64_t next_random() {  // xorshift64*
    g_state ^= g_state >> 12;
    g_state ^= g_state << 25;
    g_state ^= g_state >> 27;
    return g_state * 0x2545f4914f6cdd1dull;
}

uint64_t g_checked = 0;

void check(const std::vector<uint8_t> &bytes) {
    // An exact-size heap copy (a zero-length input gets a one-byte buffer it
    // is not allowed to read).
    uint8_t *buf = static_cast<uint8_t *>(malloc(bytes.empty() ? 1 : bytes.size()));
    if (!bytes.empty()) memcpy(buf, bytes.data(), bytes.size());
    uint32_t count = 0;
    const int32_t status = qwh_shard_validate(buf, bytes.size(), &count);
    (void)qwh_shard_verify_checksum(buf, bytes.size());
    qwh_tensor_entry entry;
    for (uint16_t kind = 0; kind < 48; kind += 3)
        for (uint16_t layer : {0, 1, 2, 1024})
            if (qwh_shard_find(buf, bytes.size(), kind, layer, &entry) == QWH_OK && status == QWH_OK) {
                // A found entry of a valid shard lies inside the buffer.
                if (entry.offset_bytes > bytes.size() || entry.len_bytes > bytes.size()) abort();
            }
    qwh_model_config config;
    uint32_t reason = 0;
    if (qwh_config_parse(buf, bytes.size(), &config, &reason) == QWH_OK) {
        qwh_decoder_config dims;
        (void)qwh_config_decoder(&config, &dims);
    }
    free(buf);
    ++g_checked;
}

void mutate_and_check(const std::vector<uint8_t> &base, int mutations) {
    check(base);
    for (int m = 0; m < mutations; ++m) {
        std::vector<uint8_t> b = base;
        const uint64_t r = next_random();
        const size_t n = b.size();
        switch (r % 6) {
        case 0:  // flip a few bytes
            for (int i = 0; i < 1 + (int)(r >> 8) % 4 && n; ++i) b[next_random() % n] ^= (uint8_t)(1 + next_random() % 255);
            break;
        case 1:  // an aligned 32-bit field to an extreme value
            if (n >= 4) {
                static const uint32_t values[] = {0u, 1u, 0x7fffffffu, 0x80000000u, 0xffffffffu, 0x10000u, 0xfffffff0u};
                const uint32_t v = values[next_random() % 7];
                memcpy(&b[(next_random() % (n / 4)) * 4], &v, 4);
            }
            break;
        case 2:  // an aligned 64-bit field to an extreme value
            if (n >= 8) {
                static const uint64_t values[] = {0ull, ~0ull, 1ull << 63, (1ull << 32) - 1, 1ull << 40};
                const uint64_t v = values[next_random() % 5];
                memcpy(&b[(next_random() % (n / 8)) * 8], &v, 8);
            }
            break;
        case 3:  // truncate
            b.resize(n ? next_random() % n : 0);
            break;
        case 4:  // append bytes
            for (int i = 0; i < 1 + (int)(next_random() % 64); ++i) b.push_back((uint8_t)next_random());
            break;
        default:  // a field of an index entry (40 bytes from the index start)
            if (n >= 32 + 40) {
                const size_t at = 32 + 40 * (next_random() % ((n - 32) / 40)) + 4 * (next_random() % 10);
                const uint32_t v = (uint32_t)next_random();
                if (at + 4 <= n) memcpy(&b[at], &v, 4);
            }
            break;
        }
        check(b);
    }
}

}  // namespace

int main(int argc, char **argv) {
    if (argc < 3) {
        fprintf(stderr, "usage: %s <mutations per file> <file>...\n", argv[0]);
        return 2;
    }
    const int mutations = atoi(argv[1]);
    for (int i = 2; i < argc; ++i) {
        FILE *f = fopen(argv[i], "rb");
        if (!f) {
            fprintf(stderr, "cannot open %s\n", argv[i]);
            return 2;
        }
        std::vector<uint8_t> bytes;
        int c;
        while ((c = fgetc(f)) != EOF) bytes.push_back((uint8_t)c);
        fclose(f);
        mutate_and_check(bytes, mutations);
    }
    printf("checked %llu inputs\n", (unsigned long long)g_checked);
    return 0;
}
