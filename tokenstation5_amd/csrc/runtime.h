// Internal host-side state of libts5hip.so: the context, error reporting.
#pragma once
#include <hip/hip_runtime_api.h>

#include <cstdarg>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/ts5hip.h"

struct ts5hip_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    std::vector<hipEvent_t> marks;  // ts5hip_timer_mark's events, made on first use
    std::string err;
    int n_cu = 0;
    std::string arch;
    int64_t hbm = 0;
    // Scratch of the per-op entry points (attention partials, reductions),
    // grown on demand outside any graph capture.
    void *scratch = nullptr;
    size_t scratch_bytes = 0;
    // Zeroed once; kernels that count finished workgroups leave them zero.
    int *counters = nullptr;  // 4096 attention counters (CTR_STRIDE apart), then the head argmax's
    // The device's no-allocation scratch (attention.hip `scratch`), looked up at init.
    void *noalloc = nullptr;
};

namespace ts5hip {

// Sets the error of ctx (or of the calling thread) and returns code.
int fail(ts5hip_ctx *ctx, int code, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
int hip_fail(ts5hip_ctx *ctx, hipError_t e, const char *what);
// Grows ctx->scratch to at least `bytes`.
int ensure_scratch(ts5hip_ctx *ctx, size_t bytes);

}  // namespace ts5hip

#define TS5_HIP(ctx, call)                                                 \
    do {                                                                   \
        hipError_t e_ = (call);                                            \
        if (e_ != hipSuccess) return ts5hip::hip_fail((ctx), e_, #call); \
    } while (0)
