// The context, device-memory plumbing, weight formats and per-op entry
// points of the C ABI (include/ts5hip.h). Host code; kernels are reached
// through the launchers of kernels.h.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <random>
#include <vector>

#include "common_host.h"
#include "kernels.h"
#include "runtime.h"

using namespace ts5hip;

namespace {
thread_local std::string g_thread_err;
// The per-op entry points' completion counters: up to 4096 (query, KV head)
// attention merges, then the head argmax's.
constexpr size_t CTX_COUNTER_INTS = 4096 * CTR_STRIDE + ARGMAX_CTR_INTS;
}

namespace ts5hip {

int fail(ts5hip_ctx *ctx, int code, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    (ctx ? ctx->err : g_thread_err) = buf;
    return code;
}

int hip_fail(ts5hip_ctx *ctx, hipError_t e, const char *what) {
    return fail(ctx, TS5HIP_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

int upload_weight(ts5hip_ctx *ctx, uint32_t t, int64_t ne0, int64_t nrows, const void *gguf, void *dst, int64_t row0,
                  int64_t total_rows) {
    const uint32_t dt = device_type(t);
    const SplitDst d = split_dst(dt, ne0, total_rows, dst, row0);
    const int64_t nblocks = ne0 / block_values(t) * nrows;  // GGUF blocks
    const size_t src_bytes = (size_t)nblocks * gguf_block_bytes(t);
    if (!split_layout(dt)) return ts5hip_upload(ctx, d.body, gguf, src_bytes);
    // Split layouts: stage the GGUF blocks in HBM, then repack on the device.
    void *tmp = nullptr;
    TS5_HIP(ctx, hipMalloc(&tmp, src_bytes));
    hipError_t e = hipMemcpyAsync(tmp, gguf, src_bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = launch_repack(t, nblocks, tmp, d.body, d.scales, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(tmp);
    if (e != hipSuccess) return hip_fail(ctx, e, "weight upload");
    return TS5HIP_OK;
}

int ensure_scratch(ts5hip_ctx *ctx, size_t bytes) {
    if (ctx->scratch_bytes >= bytes) return TS5HIP_OK;
    if (ctx->scratch) {
        TS5_HIP(ctx, hipStreamSynchronize(ctx->stream));
        TS5_HIP(ctx, hipFree(ctx->scratch));
        ctx->scratch = nullptr;
        ctx->scratch_bytes = 0;
    }
    bytes = align_up(bytes, 1 << 20);
    TS5_HIP(ctx, hipMalloc(&ctx->scratch, bytes));
    ctx->scratch_bytes = bytes;
    return TS5HIP_OK;
}

}  // namespace ts5hip

extern "C" {

const char *ts5hip_last_error(const ts5hip_ctx *ctx) { return ctx ? ctx->err.c_str() : g_thread_err.c_str(); }

int ts5hip_init(int device, ts5hip_ctx **out) {
    if (!out) return fail(nullptr, TS5HIP_ERR_ARG, "out is null");
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n == 0) return fail(nullptr, TS5HIP_ERR_HIP, "no HIP device (%s)", hipGetErrorString(e));
    if (device < 0 || device >= n) return fail(nullptr, TS5HIP_ERR_ARG, "device %d of %d", device, n);
    hipDeviceProp_t p;
    if ((e = hipGetDeviceProperties(&p, device)) != hipSuccess) return hip_fail(nullptr, e, "hipGetDeviceProperties");
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(nullptr, TS5HIP_ERR_UNSUPPORTED, "device %d is %s; this library is built for gfx950", device,
                    p.gcnArchName);
    if ((e = hipSetDevice(device)) != hipSuccess) return hip_fail(nullptr, e, "hipSetDevice");
    ts5hip_ctx *c = new ts5hip_ctx();
    c->device = device;
    c->n_cu = p.multiProcessorCount;
    c->arch = p.gcnArchName;
    c->hbm = (int64_t)p.totalGlobalMem;
    set_gemm_cu_count(c->n_cu);
    set_cu_count(c->n_cu);
    if ((e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking)) != hipSuccess ||
        (e = hipEventCreate(&c->ev0)) != hipSuccess || (e = hipEventCreate(&c->ev1)) != hipSuccess ||
        (e = hipMalloc((void **)&c->counters, CTX_COUNTER_INTS * sizeof(int))) != hipSuccess ||
        (e = hipMemset(c->counters, 0, CTX_COUNTER_INTS * sizeof(int))) != hipSuccess) {
        hip_fail(nullptr, e, "stream/event creation");
        ts5hip_destroy(c);
        return TS5HIP_ERR_HIP;
    }
    if ((e = attn_noalloc_setup(device, &c->noalloc, c->stream)) != hipSuccess) {
        hip_fail(nullptr, e, "no-allocation scratch (hipGetSymbolAddress)");
        ts5hip_destroy(c);
        return TS5HIP_ERR_HIP;
    }
    *out = c;
    return TS5HIP_OK;
}

void ts5hip_destroy(ts5hip_ctx *ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    if (ctx->scratch) (void)hipFree(ctx->scratch);
    if (ctx->counters) (void)hipFree(ctx->counters);
    if (ctx->ev0) (void)hipEventDestroy(ctx->ev0);
    if (ctx->ev1) (void)hipEventDestroy(ctx->ev1);
    for (hipEvent_t e : ctx->marks) (void)hipEventDestroy(e);
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
}

int ts5hip_device_info(ts5hip_ctx *ctx, int *n_cu, char *arch, int arch_len, int64_t *hbm_bytes) {
    if (!ctx) return fail(nullptr, TS5HIP_ERR_ARG, "ctx is null");
    if (n_cu) *n_cu = ctx->n_cu;
    if (arch && arch_len > 0) {
        std::strncpy(arch, ctx->arch.c_str(), (size_t)arch_len - 1);
        arch[arch_len - 1] = 0;
    }
    if (hbm_bytes) *hbm_bytes = ctx->hbm;
    return TS5HIP_OK;
}

// ---- memory -------------------------------------------------------------------
int ts5hip_alloc(ts5hip_ctx *ctx, size_t bytes, void **dptr) {
    if (!ctx || !dptr) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    TS5_HIP(ctx, hipMalloc(dptr, bytes ? bytes : 1));
    return TS5HIP_OK;
}
int ts5hip_free(ts5hip_ctx *ctx, void *dptr) {
    if (!ctx) return fail(nullptr, TS5HIP_ERR_ARG, "ctx is null");
    TS5_HIP(ctx, hipStreamSynchronize(ctx->stream));
    TS5_HIP(ctx, hipFree(dptr));
    return TS5HIP_OK;
}
int ts5hip_upload(ts5hip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx) return fail(nullptr, TS5HIP_ERR_ARG, "ctx is null");
    TS5_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    TS5_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TS5HIP_OK;
}
int ts5hip_download(ts5hip_ctx *ctx, void *dst, const void *src, size_t bytes) {
    if (!ctx) return fail(nullptr, TS5HIP_ERR_ARG, "ctx is null");
    TS5_HIP(ctx, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    TS5_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TS5HIP_OK;
}
int ts5hip_memset(ts5hip_ctx *ctx, void *dst, int value, size_t bytes) {
    if (!ctx) return fail(nullptr, TS5HIP_ERR_ARG, "ctx is null");
    TS5_HIP(ctx, hipMemsetAsync(dst, value, bytes, ctx->stream));
    return TS5HIP_OK;
}
int ts5hip_sync(ts5hip_ctx *ctx) {
    if (!ctx) return fail(nullptr, TS5HIP_ERR_ARG, "ctx is null");
    TS5_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TS5HIP_OK;
}
int ts5hip_timer_begin(ts5hip_ctx *ctx) {
    if (!ctx) return fail(nullptr, TS5HIP_ERR_ARG, "ctx is null");
    TS5_HIP(ctx, hipEventRecord(ctx->ev0, ctx->stream));
    return TS5HIP_OK;
}
int ts5hip_timer_mark(ts5hip_ctx *ctx, int i) {
    if (!ctx || i < 0 || i >= 4096) return fail(ctx, TS5HIP_ERR_ARG, "mark %d of at most 4096", i);
    while ((int)ctx->marks.size() <= i) {
        hipEvent_t e;
        TS5_HIP(ctx, hipEventCreate(&e));
        ctx->marks.push_back(e);
    }
    TS5_HIP(ctx, hipEventRecord(ctx->marks[(size_t)i], ctx->stream));
    return TS5HIP_OK;
}
int ts5hip_timer_marks(ts5hip_ctx *ctx, int n, float *ms) {
    if (!ctx || !ms || n < 2 || n > (int)ctx->marks.size()) return fail(ctx, TS5HIP_ERR_ARG, "%d marks", n);
    TS5_HIP(ctx, hipEventSynchronize(ctx->marks[(size_t)n - 1]));
    for (int i = 0; i + 1 < n; i++) TS5_HIP(ctx, hipEventElapsedTime(ms + i, ctx->marks[(size_t)i], ctx->marks[(size_t)i + 1]));
    return TS5HIP_OK;
}
int ts5hip_timer_end(ts5hip_ctx *ctx, float *ms) {
    if (!ctx || !ms) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    TS5_HIP(ctx, hipEventRecord(ctx->ev1, ctx->stream));
    TS5_HIP(ctx, hipEventSynchronize(ctx->ev1));
    TS5_HIP(ctx, hipEventElapsedTime(ms, ctx->ev0, ctx->ev1));
    return TS5HIP_OK;
}

// ---- weights ------------------------------------------------------------------
int ts5hip_supports_type(uint32_t type) {
    switch (type) {
    case T_F32: case T_F16: case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: case T_Q8_0: case T_Q4_K:
    case T_Q5_K: case T_Q6_K: return 1;
    }
    return 0;
}

int64_t ts5hip_weight_bytes(uint32_t type, int64_t ne0, int64_t ne1) {
    if (ne0 <= 0 || ne1 <= 0) return -1;
    const size_t b = device_bytes(type, ne0, ne1);
    return b ? (int64_t)b : -1;
}

int ts5hip_weight_upload(ts5hip_ctx *ctx, uint32_t type, int64_t ne0, int64_t ne1, const void *gguf, void *dst) {
    if (!ctx || !gguf || !dst) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (ts5hip_weight_bytes(type, ne0, ne1) < 0)
        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "type %u with %lld x %lld", type, (long long)ne0, (long long)ne1);
    return upload_weight(ctx, type, ne0, ne1, gguf, dst, 0, ne1);
}

int ts5hip_weight_synth(ts5hip_ctx *ctx, uint32_t type, int64_t ne0, int64_t ne1, uint64_t seed, int centered,
                        void *dst) {
    if (!ctx || !dst) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (ts5hip_weight_bytes(type, ne0, ne1) < 0 || device_type(type) != type)
        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "synthetic type %u with %lld x %lld", type, (long long)ne0, (long long)ne1);
    const SplitDst d = split_dst(type, ne0, ne1, dst, 0);
    TS5_HIP(ctx, launch_synth(type, ne0, ne1, seed, centered, d.body, d.scales, ctx->stream));
    return TS5HIP_OK;
}

int ts5hip_kv_synth(ts5hip_ctx *ctx, uint64_t seed, int64_t n, int kv_type, void *values, void *scales) {
    if (!ctx || !values || (kv_type == KV_Q8 && !scales)) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (n <= 0 || n % 32 || (kv_type != KV_Q8 && kv_type != KV_F16))
        return fail(ctx, TS5HIP_ERR_ARG, "n %lld (a multiple of 32), cache type %d (q8 or f16)", (long long)n, kv_type);
    TS5_HIP(ctx, launch_kv_synth(n, seed, kv_type == KV_F16, values, scales, ctx->stream));
    return TS5HIP_OK;
}

// ---- per-op entry points ----------------------------------------------------------
int ts5hip_dequantize(ts5hip_ctx *ctx, uint32_t type, const void *w, int64_t ne0, int64_t rows, float *y) {
    if (!ctx || !w || !y) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (type != T_F32 && type != T_F16 && ts5hip_weight_bytes(type, ne0, rows) < 0)
        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "type %u with ne0 %lld", type, (long long)ne0);
    TS5_HIP(ctx, launch_dequant(device_type(type), w, ne0, rows, y, ctx->stream));
    return TS5HIP_OK;
}

int64_t ts5hip_act_bytes(int64_t n) { return n > 0 && n % 32 == 0 ? (int64_t)act_bytes(n) : -1; }

int ts5hip_act_quantize(ts5hip_ctx *ctx, const float *x, const float *norm_w, float eps, int64_t n, int ntok,
                        void *act) {
    if (!ctx || !x || !act) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (n <= 0 || n % 32 || ntok <= 0) return fail(ctx, TS5HIP_ERR_ARG, "n %lld (a multiple of 32), ntok %d", (long long)n, ntok);
    TS5_HIP(ctx, launch_act_quant(x, n, norm_w, eps, (int)n, ntok, act, ctx->stream));
    return TS5HIP_OK;
}

int ts5hip_rmsnorm(ts5hip_ctx *ctx, const float *x, const float *w, float eps, int64_t n, int ntok, float *y) {
    if (!ctx || !x || !w || !y) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (n <= 0 || ntok <= 0) return fail(ctx, TS5HIP_ERR_ARG, "bad shape");
    TS5_HIP(ctx, launch_rmsnorm(x, w, eps, (int)n, ntok, y, ctx->stream));
    return TS5HIP_OK;
}

static int check_matrix(ts5hip_ctx *ctx, uint32_t type, int64_t ne0, int64_t ne1) {
    if (!ts5hip_supports_type(type) || ts5hip_weight_bytes(type, ne0, ne1) < 0)
        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "matvec of type %u, %lld x %lld", type, (long long)ne1,
                    (long long)ne0);
    if (ne0 > 16384) return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "input of %lld values (at most 16384)", (long long)ne0);
    if (ne0 % 32) return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "rows of %lld values (a multiple of 32)", (long long)ne0);
    return TS5HIP_OK;
}

int ts5hip_matvec(ts5hip_ctx *ctx, uint32_t type, const void *w, int64_t ne0, int64_t ne1, const float *x,
                  const float *norm_w, float eps, float *y, int accumulate) {
    if (!ctx || !w || !x || !y) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (int rc = check_matrix(ctx, type, ne0, ne1)) return rc;
    TS5_HIP(ctx, launch_matvec(device_type(type), w, ne0, ne1, x, norm_w, eps, y, accumulate, ctx->stream));
    return TS5HIP_OK;
}

int ts5hip_matvec_glu(ts5hip_ctx *ctx, uint32_t type, const void *w_gate, const void *w_up, int64_t ne0, int64_t ne1,
                      const float *x, const float *norm_w, float eps, float *y) {
    if (!ctx || !w_gate || !w_up || !x || !y) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (int rc = check_matrix(ctx, type, ne0, ne1)) return rc;
    TS5_HIP(ctx, launch_matvec_glu(device_type(type), w_gate, w_up, ne0, ne1, x, norm_w, eps, y, ctx->stream));
    return TS5HIP_OK;
}

// Several tokens: their activations, then the matrix-core matmul.
static int matmul_any(ts5hip_ctx *ctx, uint32_t type, const void *w, const void *w2, int64_t ne0, int64_t ne1,
                      const float *x, int ntok, const float *norm_w, float eps, float *y, int mode) {
    if (!ctx || !w || !x || !y || (mode == 2 && !w2)) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (ntok < 1 || ntok > 4096) return fail(ctx, TS5HIP_ERR_ARG, "ntok %d outside 1..4096", ntok);
    if (int rc = check_matrix(ctx, type, ne0, ne1)) return rc;
    type = device_type(type);
    if (type == T_F16 || type == T_F32) {
        TS5_HIP(ctx, launch_matvec_tokens(type, w, w2, ne0, ne1, x, ne0, norm_w, eps, ntok, mode, y, ne1, ctx->stream));
        return TS5HIP_OK;
    }
    if (gemm_fused_fits(type, ne0, ntok)) {
        TS5_HIP(ctx, launch_gemm_fused(w, w2, ne0, ne1, x, ne0, norm_w, eps, ntok, mode, y, y, ne1, ctx->stream));
        return TS5HIP_OK;
    }
    const size_t act = align_up((size_t)ntok * gemm_act_bytes(type, ne0, ntok), 256);
    const size_t part = gemm_scratch_bytes(ne1, ntok, (int)(ne0 / block_values(type)));
    if (int rc = ensure_scratch(ctx, act + part)) return rc;
    uint8_t *base = (uint8_t *)ctx->scratch;
    TS5_HIP(ctx, launch_gemm_act(type, x, ne0, norm_w, eps, (int)ne0, ntok, base, ctx->stream));
    TS5_HIP(ctx, launch_gemm(type, w, w2, ne0, ne1, base, ntok, mode, y, y, ne1, base + act, ctx->stream));
    return TS5HIP_OK;
}

int ts5hip_matmul(ts5hip_ctx *ctx, uint32_t type, const void *w, int64_t ne0, int64_t ne1, const float *x, int ntok,
                  const float *norm_w, float eps, float *y, int accumulate) {
    return matmul_any(ctx, type, w, nullptr, ne0, ne1, x, ntok, norm_w, eps, y, accumulate ? 1 : 0);
}

int ts5hip_matmul_glu(ts5hip_ctx *ctx, uint32_t type, const void *w_gate, const void *w_up, int64_t ne0, int64_t ne1,
                      const float *x, int ntok, const float *norm_w, float eps, float *y) {
    return matmul_any(ctx, type, w_gate, w_up, ne0, ne1, x, ntok, norm_w, eps, y, 2);
}

int ts5hip_matvec_argmax(ts5hip_ctx *ctx, uint32_t type, const void *w, int64_t ne0, int64_t ne1, const float *x,
                         const float *norm_w, float eps, float *y, int32_t *out_dev) {
    if (!ctx || !w || !x || !y || !out_dev) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (int rc = check_matrix(ctx, type, ne0, ne1)) return rc;
    if (int rc = ensure_scratch(ctx, matvec_argmax_scratch_bytes())) return rc;
    TS5_HIP(ctx, launch_matvec_argmax(device_type(type), w, ne0, ne1, x, norm_w, eps, y, ctx->scratch, ctx->counters + 4096 * CTR_STRIDE,
                                      out_dev, nullptr, nullptr, ctx->stream));
    return TS5HIP_OK;
}

int ts5hip_rope_table(ts5hip_ctx *ctx, int n_rot, int n_pos, float base, float scale, const float *freqs_host,
                      float *dst) {
    if (!ctx || !dst || n_rot <= 0 || n_rot % 2 || n_pos <= 0) return fail(ctx, TS5HIP_ERR_ARG, "bad argument");
    std::vector<float> t;
    rope_table_host(n_rot, n_pos, base, scale, freqs_host, t);
    return ts5hip_upload(ctx, dst, t.data(), t.size() * sizeof(float));
}

int ts5hip_rope_kv_append(ts5hip_ctx *ctx, const float *qkv, int ntok, const int32_t *pos0_dev, int n_head,
                          int n_head_kv, int head_dim, int n_rot, int neox, const float *rope_cs, int n_ctx,
                          const float *bias, const float *q_norm, const float *k_norm, float eps, float *q_out,
                          void *k8, void *ks, void *v8, void *vs) {
    if (!ctx || !qkv || !pos0_dev || !rope_cs || !q_out || !k8 || !ks || !v8 || !vs)
        return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (ntok <= 0 || n_head_kv <= 0 || n_head % n_head_kv || (head_dim != 64 && head_dim != 128) || n_rot > head_dim ||
        n_rot % 2 || n_ctx <= 0)
        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "rope/kv for %d/%d heads of %d (n_rot %d)", n_head, n_head_kv,
                    head_dim, n_rot);
    const KvLayer kv{(int8_t *)k8, (uint16_t *)ks, (int8_t *)v8, (uint16_t *)vs};
    TS5_HIP(ctx, launch_rope_kv(qkv, (int64_t)(n_head + 2 * n_head_kv) * head_dim, bias, q_norm, k_norm, eps, rope_cs,
                                n_rot, neox, pos0_dev, n_head, n_head_kv, head_dim, n_ctx, ntok, q_out, kv, 0,
                                ctx->stream));
    return TS5HIP_OK;
}

// The split-K decode attention with its partials and merge counters at
// `part` / `counters`, or (null) in the context's growable scratch.
static int attn_decode_into(ts5hip_ctx *ctx, const float *q, int B, int n_head, int n_head_kv, int head_dim,
                            const void *k8, const void *ks, const void *v8, const void *vs, int n_ctx,
                            const int32_t *n_keys_dev, int kv_per_batch, float scale, int n_split, float *out,
                            float *part, int *counters, int kv_f16 = 0) {
    if (!ctx || !q || !k8 || !v8 || (!kv_f16 && (!ks || !vs)) || !n_keys_dev || !out)
        return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (B <= 0 || n_ctx <= 0 || !attn_supported(n_head, n_head_kv, head_dim))
        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "attention for %d/%d heads of %d", n_head, n_head_kv, head_dim);
    if (B * n_head_kv > 4096) return fail(ctx, TS5HIP_ERR_ARG, "batch of %d x %d KV heads", B, n_head_kv);
    if (n_split <= 0) n_split = attn_splits(B, n_head_kv, ctx->n_cu);
    if (n_split > 64) return fail(ctx, TS5HIP_ERR_ARG, "n_split %d (at most 64)", n_split);
    const size_t need = attn_partial_bytes(B, n_split, n_head, n_head_kv, head_dim);
    if (part) {
        if (need > NOALLOC_BYTES - NOALLOC_COUNTER_BYTES)
            return fail(ctx, TS5HIP_ERR_ARG,
                        "%d queries x %d splits x %d KV heads need %zu bytes of partials; the no-allocation "
                        "scratch holds %zu",
                        B, n_split, n_head_kv, need, NOALLOC_BYTES - NOALLOC_COUNTER_BYTES);
    } else {
        if (int rc = ensure_scratch(ctx, need)) return rc;
        part = (float *)ctx->scratch, counters = ctx->counters;
    }
    AttnIO io{};
    io.q = q, io.q_stride = (int64_t)n_head * head_dim, io.rope = 0, io.append = 0;
    io.kv = KvLayer{(int8_t *)k8, (uint16_t *)ks, (int8_t *)v8, (uint16_t *)vs};
    io.kv_f16 = kv_f16;
    io.kv_per_batch = kv_per_batch, io.n_ctx = n_ctx, io.n_keys = n_keys_dev;
    io.B = B, io.H = n_head, io.HKV = n_head_kv, io.HD = head_dim, io.n_split = n_split, io.scale = scale;
    io.part = part, io.counters = counters, io.out = out;
    TS5_HIP(ctx, launch_attn(io, ctx->stream));
    return TS5HIP_OK;
}

int ts5hip_attn_decode(ts5hip_ctx *ctx, const float *q, int B, int n_head, int n_head_kv, int head_dim,
                       const void *k8, const void *ks, const void *v8, const void *vs, int n_ctx,
                       const int32_t *n_keys_dev, int kv_per_batch, float scale, int n_split, float *out) {
    return attn_decode_into(ctx, q, B, n_head, n_head_kv, head_dim, k8, ks, v8, vs, n_ctx, n_keys_dev, kv_per_batch,
                            scale, n_split, out, nullptr, nullptr);
}

int ts5hip_attn_decode_f16(ts5hip_ctx *ctx, const float *q, int B, int n_head, int n_head_kv, int head_dim,
                           const void *k16, const void *v16, int n_ctx, const int32_t *n_keys_dev, int kv_per_batch,
                           float scale, int n_split, float *out) {
    return attn_decode_into(ctx, q, B, n_head, n_head_kv, head_dim, k16, nullptr, v16, nullptr, n_ctx, n_keys_dev,
                            kv_per_batch, scale, n_split, out, nullptr, nullptr, 1);
}

int ts5hip_attn_decode_noalloc(ts5hip_ctx *ctx, const float *q, int B, int n_head, int n_head_kv, int head_dim,
                               const void *k8, const void *ks, const void *v8, const void *vs, int n_ctx,
                               const int32_t *n_keys_dev, int kv_per_batch, float scale, int n_split, float *out) {
    if (!ctx || !ctx->noalloc) return fail(ctx, TS5HIP_ERR_STATE, "no context or no-allocation scratch");
    uint8_t *base = (uint8_t *)ctx->noalloc;
    return attn_decode_into(ctx, q, B, n_head, n_head_kv, head_dim, k8, ks, v8, vs, n_ctx, n_keys_dev, kv_per_batch,
                            scale, n_split, out, (float *)(base + NOALLOC_COUNTER_BYTES), (int *)base);
}

static int attn_prompt_into(ts5hip_ctx *ctx, const float *q, int nq, int n_head, int n_head_kv, int head_dim,
                            const void *k, const void *ks, const void *v, const void *vs, int kv_f16, int n_ctx,
                            int pos0, float scale, float *out) {
    if (!ctx || !q || !k || !v || !out || (!kv_f16 && (!ks || !vs))) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (!attn_prefill_supported(n_head, n_head_kv, head_dim))
        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "prompt attention for %d/%d heads of %d", n_head, n_head_kv, head_dim);
    if (nq <= 0 || pos0 < 0 || n_ctx <= 0 || (int64_t)pos0 + nq > n_ctx)
        return fail(ctx, TS5HIP_ERR_ARG, "%d queries at %d in a cache of %d", nq, pos0, n_ctx);
    if (int rc = ensure_scratch(ctx, attn_prefill_partial_bytes(nq, n_head, head_dim, (int64_t)pos0 + nq))) return rc;
    const KvLayer kv{(int8_t *)k, (uint16_t *)ks, (int8_t *)v, (uint16_t *)vs};
    TS5_HIP(ctx, launch_attn_prefill(q, (int64_t)n_head * head_dim, kv, kv_f16, n_ctx, n_head, n_head_kv, head_dim,
                                     pos0, nq, scale, (float *)ctx->scratch, out, ctx->stream));
    return TS5HIP_OK;
}

int ts5hip_attn_prompt(ts5hip_ctx *ctx, const float *q, int nq, int n_head, int n_head_kv, int head_dim,
                       const void *k8, const void *ks, const void *v8, const void *vs, int n_ctx, int pos0,
                       float scale, float *out) {
    return attn_prompt_into(ctx, q, nq, n_head, n_head_kv, head_dim, k8, ks, v8, vs, 0, n_ctx, pos0, scale, out);
}

int ts5hip_attn_prompt_f16(ts5hip_ctx *ctx, const float *q, int nq, int n_head, int n_head_kv, int head_dim,
                           const void *k16, const void *v16, int n_ctx, int pos0, float scale, float *out) {
    return attn_prompt_into(ctx, q, nq, n_head, n_head_kv, head_dim, k16, nullptr, v16, nullptr, 1, n_ctx, pos0, scale,
                            out);
}

int ts5hip_argmax(ts5hip_ctx *ctx, const float *x, int n, int rows, int32_t *out_dev) {
    if (!ctx || !x || !out_dev || n <= 0 || rows <= 0) return fail(ctx, TS5HIP_ERR_ARG, "bad argument");
    if (int rc = ensure_scratch(ctx, argmax_scratch_bytes(rows))) return rc;
    TS5_HIP(ctx, launch_argmax(x, n, rows, ctx->scratch, out_dev, nullptr, nullptr, ctx->stream));
    return TS5HIP_OK;
}

int ts5hip_topk(ts5hip_ctx *ctx, const float *x, int n, int k, float *vals_dev, int32_t *ids_dev) {
    if (!ctx || !x || !vals_dev || !ids_dev) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    if (k <= 0 || k > topk_max() || n < k || n > topk_max_n())
        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "top-%d of %d (k <= %d, n <= %d)", k, n, topk_max(), topk_max_n());
    if (int rc = ensure_scratch(ctx, topk_scratch_bytes(1))) return rc;
    TS5_HIP(ctx, launch_topk(x, n, k, 1, ctx->scratch, vals_dev, ids_dev, ctx->stream));
    return TS5HIP_OK;
}

// ---- sampler --------------------------------------------------------------------------
struct ts5hip_sampler {
    std::mt19937_64 rng;
    std::vector<int32_t> heap;
    std::vector<double> w;
};

ts5hip_sampler *ts5hip_sampler_new(uint64_t seed) {
    ts5hip_sampler *s = new ts5hip_sampler();
    s->rng.seed(seed);
    return s;
}

void ts5hip_sampler_free(ts5hip_sampler *s) { delete s; }

int32_t ts5hip_sampler_draw(ts5hip_sampler *s, const int32_t *ids, const float *logits, int k, float temperature,
                            float top_p) {
    if (!s || !ids || !logits || k <= 0) return -1;
    return sampler_draw(s->rng, s->w, ids, logits, k, temperature, top_p);
}

}  // extern "C"

namespace ts5hip {

void sampler_reseed(ts5hip_sampler *s, uint64_t seed) { s->rng.seed(seed); }

// Engine::sample (engine/src/engine.cpp:16-46) over a host row of n logits.
int32_t sample_host_row(ts5hip_sampler *s, const float *lg, int n, float temperature, float top_p, int top_k) {
    if (temperature <= 0) return (int32_t)(std::max_element(lg, lg + n) - lg);
    const int k = top_k > 0 ? std::min(top_k, n) : n;
    auto above = [lg](int32_t a, int32_t b) { return lg[a] > lg[b]; };  // heap front: smallest kept
    std::vector<int32_t> &h = s->heap;
    h.clear();
    for (int32_t i = 0; i < n; i++) {
        if ((int)h.size() < k) {
            h.push_back(i);
            std::push_heap(h.begin(), h.end(), above);
        } else if (lg[i] > lg[h.front()]) {
            std::pop_heap(h.begin(), h.end(), above);
            h.back() = i;
            std::push_heap(h.begin(), h.end(), above);
        }
    }
    std::sort_heap(h.begin(), h.end(), above);
    std::vector<float> cand(h.size());
    for (size_t i = 0; i < h.size(); i++) cand[i] = lg[h[i]];
    return sampler_draw(s->rng, s->w, h.data(), cand.data(), k, temperature, top_p);
}

}  // namespace ts5hip
