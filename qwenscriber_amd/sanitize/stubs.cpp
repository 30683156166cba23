// Link stand-ins for the sanitized host build of the parsers: the device
// paths of shard.cpp (qwh_shard_load and the functions that use a loaded
// shard) reference the HIP runtime and capi.cpp's helpers, which the parser
// checks never call. Each stand-in reports failure.
#include <cstdarg>
#include <cstdio>

#include "../csrc/common.h"

namespace qwh {

int32_t fail(qwh_ctx *ctx, int32_t status, const char *fmt, ...) {
    if (ctx) {
        char buf[256];
        va_list args;
        va_start(args, fmt);
        vsnprintf(buf, sizeof buf, fmt, args);
        va_end(args);
        ctx->last_error = buf;
    }
    return status;
}

int32_t check_hip(qwh_ctx *, hipError_t err, const char *) { return err == hipSuccess ? QWH_OK : QWH_E_DEVICE; }

uint64_t add_matrix(qwh_ctx *, const Matrix &) { return 0; }

}  // namespace qwh

extern "C" {
hipError_t hipMalloc(void **, size_t) { return hipErrorNotSupported; }
hipError_t hipFree(void *) { return hipErrorNotSupported; }
hipError_t hipMemcpyAsync(void *, const void *, size_t, hipMemcpyKind, hipStream_t) { return hipErrorNotSupported; }
hipError_t hipStreamSynchronize(hipStream_t) { return hipErrorNotSupported; }
}
