// Decode attention over a q8 KV cache.
//
//  k_rope_kv      per (head, token): bias, optional per-head RMSNorm, RoPE
//                 (engine/src/cpu_backend.cpp:57-68, :198-221), then for K and
//                 V heads the q8 rounding of round_kv (:78-90) written as int8
//                 quants + f16 scales (the split layout of qkv_post.glsl:29-41).
//                 (kept for prompt chunks: their K/V must all be in the
//                 cache before any of them attends).
//  k_attn_lds,    split-K flash decode: per (key slice, KV head, query) one
//  k_attn         workgroup scores its G = H/HKV query heads against 64-key
//                 tiles with an online softmax (attn.glsl:54-162); it also
//                 does the RoPE and q8 append of the new keys in its slice,
//                 and the last workgroup per (query, KV head) merges the
//                 splits (attn_merge.comp:18-47).
//  k_attn_m1      the same for one query per cache at head dimension 128
//                 (q8 or f16), its key loop on the matrix cores (attn_m1.hip).
//  k_attn_mq,     the same for a batch of 2-16 consecutive queries on one q8
//  k_attn_mq_merge cache (B x G <= 32 rows, head dimension 128): all the
//                 batch's queries in each (key slice, KV head) work item, on
//                 the matrix cores, and the splits merged by a second launch.
//
// Cache layout per layer: K8/V8 int8 [seq][kv_head][slot][head_dim] and
// Ks/Vs f16 [seq][kv_head][slot][head_dim/32]: one KV head's keys are
// contiguous, 128 + 8 bytes per key at head_dim 128.
#include <mutex>

#include "attn_lds.h"
#include "attn_mq.h"


namespace ts5hip {


__device__ inline float block_sum64(float v) { return wave_sum(v); }

// grid (H + 2*HKV, ntok), 64 threads (one wave): thread i holds values 2i, 2i+1
// (and 2i + 128, 2i + 129 at head dimension 256).
__global__ __launch_bounds__(64) void k_rope_kv(const float *__restrict__ qkv, int64_t qkv_stride,
                                                const float *__restrict__ bias, const float *__restrict__ q_norm,
                                                const float *__restrict__ k_norm, float eps,
                                                const float2 *__restrict__ rope_cs, int n_rot, int neox,
                                                const int32_t *__restrict__ pos0p, int H, int HKV, int HD,
                                                int n_ctx, float *__restrict__ q_out, KvLayer kv, int kv_f16) {
    __shared__ float v[256];
    const int hh = blockIdx.x, t = blockIdx.y, i = threadIdx.x;
    const int pos = pos0p[0] + t;
    const float *src = qkv + (int64_t)t * qkv_stride + (int64_t)hh * HD;
    const bool is_q = hh < H, is_k = !is_q && hh < H + HKV;
    for (int j = i; j < HD; j += 64) v[j] = src[j] + (bias ? bias[(int64_t)hh * HD + j] : 0.f);
    __syncthreads();
    const float *nw = is_q ? q_norm : (is_k ? k_norm : nullptr);
    if (nw) {
        float ss = 0.f;
        for (int j = i; j < HD; j += 64) ss += v[j] * v[j];
        ss = block_sum64(ss);
        const float s = 1.0f / sqrtf(ss / (float)HD + eps);
        __syncthreads();
        for (int j = i; j < HD; j += 64) v[j] = v[j] * s * nw[j];
        __syncthreads();
    }
    if (is_q || is_k) {
        for (int r = i; r < n_rot / 2; r += 64) {
            const int a = neox ? r : 2 * r, b = neox ? r + n_rot / 2 : 2 * r + 1;
            const float2 cs = rope_cs[(int64_t)pos * (n_rot / 2) + r];
            float x0 = v[a], x1 = v[b];
            rope_pair(x0, x1, cs.x, cs.y);
            v[a] = x0;
            v[b] = x1;
        }
        __syncthreads();
    }
    if (is_q) {
        float *dst = q_out + ((int64_t)t * H + hh) * HD;
        for (int j = i; j < HD; j += 64) dst[j] = v[j];
        return;
    }
    const int kvh = is_k ? hh - H : hh - H - HKV;
    if (kv_f16) {  // f16: each value to the nearest half (engine/src/cpu_backend.cpp:80)
        uint16_t *c16 = (uint16_t *)(is_k ? kv.k : kv.v);
        const int64_t slot = (int64_t)kvh * n_ctx + pos;
        for (int d = 2 * i; d < HD; d += 128)
            *(uint32_t *)(c16 + slot * HD + d) = (uint32_t)f2h(v[d]) | (uint32_t)f2h(v[d + 1]) << 16;
        return;
    }
    // q8: per 32 values sc = f16(amax / 127), q = clamp(rint(v / sc), +-127).
    int8_t *q8 = is_k ? kv.k : kv.v;
    uint16_t *sc8 = is_k ? kv.ks : kv.vs;
    const int64_t slot = (int64_t)kvh * n_ctx + pos;
    for (int d = 2 * i; d < HD; d += 128) {
        float a0 = v[d], a1 = v[d + 1];
        float amax = fmaxf(fabsf(a0), fabsf(a1));
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 16));
        const uint16_t sh = f2h(amax / 127.0f);
        const float sc = h2f(sh);
        int q0 = 0, q1 = 0;
        if (sc > 0.f) {
            q0 = (int)fminf(127.f, fmaxf(-127.f, rintf(a0 / sc)));
            q1 = (int)fminf(127.f, fmaxf(-127.f, rintf(a1 / sc)));
        }
        uint16_t packed = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
        *(uint16_t *)(q8 + slot * HD + d) = packed;
        if ((i & 15) == 0) sc8[slot * (HD / 32) + d / 32] = sh;
    }
}

// What the work item needs before its first loads (where its keys are) comes
// first and one by one, 14 dwords preloaded into SGPRs at wave launch (this
// file builds with -amdgpu-kernarg-preload-count=16); the rest of AttnArgs
// (query, RoPE, norms, partials, output) follows in `tail`. flags: 1
// kv_per_batch, 2 append, 4 rope.
constexpr int ATTN_NT = 512;  // threads per work item: 8 waves, two per SIMD

// The same work item for short slices (one query, a cache of up to
// LDS_MAX_CTX positions): attn_slice_lds shares the slice through LDS.
template <int HD, int G, bool F16>
__global__ __launch_bounds__(ATTN_NT) void k_attn_lds(const int8_t *k8, const uint16_t *ks, const int8_t *v8,
                                                      const uint16_t *vs, const int32_t *n_keys, int n_ctx, int HKV,
                                                      int flags, int n_split, AttnArgs tail) {
    __shared__ LdsSliceLds<HD, G, ATTN_NT> S;
    AttnArgs a = tail;
    a.kv = KvLayer{const_cast<int8_t *>(k8), const_cast<uint16_t *>(ks), const_cast<int8_t *>(v8),
                   const_cast<uint16_t *>(vs)};
    a.n_keys = n_keys, a.n_ctx = n_ctx, a.HKV = HKV;
    a.kv_per_batch = flags & 1, a.append = (flags >> 1) & 1, a.rope = (flags >> 2) & 1;
    attn_slice_lds<HD, G, ATTN_NT, F16>(a, blockIdx.x, blockIdx.y, blockIdx.z, n_split, S);
}

template <int HD, int G, bool F16>
__global__ __launch_bounds__(ATTN_NT) void k_attn(const int8_t *k8, const uint16_t *ks, const int8_t *v8,
                                                  const uint16_t *vs, const int32_t *n_keys, int n_ctx, int HKV,
                                                  int flags, int n_split, AttnArgs tail) {
    __shared__ SliceLds<HD, G, ATTN_NT> S;
    AttnArgs a = tail;
    a.kv = KvLayer{const_cast<int8_t *>(k8), const_cast<uint16_t *>(ks), const_cast<int8_t *>(v8),
                   const_cast<uint16_t *>(vs)};
    a.n_keys = n_keys, a.n_ctx = n_ctx, a.HKV = HKV;
    a.kv_per_batch = flags & 1, a.append = (flags >> 1) & 1, a.rope = (flags >> 2) & 1;
    attn_slice<HD, G, ATTN_NT, F16>(a, blockIdx.x, blockIdx.y, blockIdx.z, n_split, S);
}

// A batch of B consecutive queries on one q8 cache, B x G <= 32 rows of
// head dimension 128: every query of the batch in one work item per (split,
// KV head), on the matrix cores (attn_mq.h).
__global__ __launch_bounds__(MQ_NT) void k_attn_mq(const int8_t *k8, const uint16_t *ks, const int8_t *v8,
                                                   const uint16_t *vs, const int32_t *n_keys, int n_ctx, int HKV,
                                                   int flags, int n_split, int G, int B, AttnArgs tail) {
    __shared__ MqLds S;
    AttnArgs a = tail;
    a.kv = KvLayer{const_cast<int8_t *>(k8), const_cast<uint16_t *>(ks), const_cast<int8_t *>(v8),
                   const_cast<uint16_t *>(vs)};
    a.n_keys = n_keys, a.n_ctx = n_ctx, a.HKV = HKV;
    a.kv_per_batch = 0, a.append = (flags >> 1) & 1, a.rope = (flags >> 2) & 1;
    attn_mq(a, G, B, blockIdx.x, blockIdx.y, n_split, S);
}
// Its splits' merge: grid (B x G rows, HKV), a thread per dimension.
__global__ __launch_bounds__(MQ_HD) void k_attn_mq_merge(const int32_t *n_keys, int n_split, int G, int B,
                                                         AttnArgs a) {
    a.n_keys = n_keys;
    attn_mq_merge(a, G, B, n_split, blockIdx.x, blockIdx.y);
}

// K (which 0) or V (1) at positions [pos0, pos0 + n) dequantized to fp32
// [n][HKV * HD] (engine/src/cpu_backend.cpp:95-97's row layout).
__global__ void k_kv_read(KvLayer kv, int which, int HKV, int HD, int n_ctx, int pos0, int n, int kv_f16,
                          float *__restrict__ out) {
    const int64_t total = (int64_t)n * HKV * HD;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int p = (int)(e / (HKV * HD)), h = (int)(e / HD % HKV), d = (int)(e % HD);
        const int64_t slot = (int64_t)h * n_ctx + pos0 + p;
        if (kv_f16) {
            out[e] = h2f(((const uint16_t *)(which ? kv.v : kv.k))[slot * HD + d]);
        } else {
            const int8_t q = (which ? kv.v : kv.k)[slot * HD + d];
            out[e] = (float)q * h2f((which ? kv.vs : kv.ks)[slot * (HD / 32) + d / 32]);
        }
    }
}

// K (which 0) or V (1) values [n][HKV * HD] (fp32) into positions
// [pos0, pos0 + n) of the cache, rounded as the cache keeps them (q8 per 32
// values as round_kv, engine/src/cpu_backend.cpp:78-90, or f16). One wave per
// (position, KV head), two values a lane.
__global__ __launch_bounds__(64) void k_kv_write(KvLayer kv, int which, int HKV, int HD, int n_ctx, int pos0,
                                                 int kv_f16, const float *__restrict__ in) {
    const int p = blockIdx.x, h = blockIdx.y;
    const float *src = in + ((int64_t)p * HKV + h) * HD;
    const int64_t slot = (int64_t)h * n_ctx + pos0 + p;
    for (int d = 2 * (int)threadIdx.x; d < HD; d += 128) {  // values d, d + 1 a lane
    const int i = d / 2;
    const float a0 = src[2 * i], a1 = src[2 * i + 1];
    if (kv_f16) {
        *(uint32_t *)((uint16_t *)(which ? kv.v : kv.k) + slot * HD + 2 * i) =
            (uint32_t)f2h(a0) | (uint32_t)f2h(a1) << 16;
        continue;
    }
    float amax = fmaxf(fabsf(a0), fabsf(a1));
#pragma unroll
    for (int o = 8; o > 0; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 16));
    const uint16_t sh = f2h(amax / 127.0f);
    const float sc = h2f(sh);
    int q0 = 0, q1 = 0;
    if (sc > 0.f) {
        q0 = (int)fminf(127.f, fmaxf(-127.f, rintf(a0 / sc)));
        q1 = (int)fminf(127.f, fmaxf(-127.f, rintf(a1 / sc)));
    }
    *(uint16_t *)((which ? kv.v : kv.k) + slot * HD + 2 * i) = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
    if ((i & 15) == 0) (which ? kv.vs : kv.ks)[slot * (HD / 32) + i / 16] = sh;
    }
}

hipError_t launch_kv_write(KvLayer kv, int which, int HKV, int HD, int n_ctx, int pos0, int n, int kv_f16,
                           const float *in, hipStream_t s) {
    hipLaunchKernelGGL(k_kv_write, dim3(n, HKV), dim3(64), 0, s, kv, which, HKV, HD, n_ctx, pos0, kv_f16, in);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// The scratch of the no-allocation entry point (ts5hip_attn_decode_noalloc):
// the merge counters (NOALLOC_COUNTER_BYTES, kept at zero between launches by
// the kernels themselves), then the split partials. Each GPU holds its own
// copy for the life of the process. Host code never passes `scratch` itself
// to a kernel (its host name is a stand-in, not a device address); it uses
// the address hipGetSymbolAddress gives for the current device.
static __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];

namespace {
std::mutex g_noalloc_mu;
void *g_noalloc[NOALLOC_DEVICES];  // the array's address on each device, once looked up
}  // namespace

hipError_t attn_noalloc_setup(int device, void **ptr, hipStream_t s) {
    if (device < 0 || device >= NOALLOC_DEVICES) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_noalloc_mu);
    if (!g_noalloc[device]) {
        void *p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));  // device `device` is current
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        if ((e = hipMemsetAsync(p, 0, NOALLOC_COUNTER_BYTES, s)) != hipSuccess) return e;
        if ((e = hipStreamSynchronize(s)) != hipSuccess) return e;
        g_noalloc[device] = p;
    }
    *ptr = g_noalloc[device];
    return hipSuccess;
}

// ---------------------------------------------------------------------------
hipError_t launch_kv_read(KvLayer kv, int which, int HKV, int HD, int n_ctx, int pos0, int n, int kv_f16, float *out,
                          hipStream_t s) {
    hipLaunchKernelGGL(k_kv_read, dim3(256), dim3(256), 0, s, kv, which, HKV, HD, n_ctx, pos0, n, kv_f16, out);
    return hipGetLastError();
}

hipError_t launch_rope_kv(const float *qkv, int64_t qkv_stride, const float *bias, const float *q_norm,
                          const float *k_norm, float eps, const float *rope_cs, int n_rot, int neox,
                          const int32_t *pos0, int H, int HKV, int HD, int n_ctx, int ntok, float *q_out, KvLayer kv,
                          int kv_f16, hipStream_t s) {
    hipLaunchKernelGGL(k_rope_kv, dim3(H + 2 * HKV, ntok), dim3(64), 0, s, qkv, qkv_stride, bias, q_norm, k_norm,
                       eps, (const float2 *)rope_cs, n_rot, neox, pos0, H, HKV, HD, n_ctx, q_out, kv, kv_f16);
    return hipGetLastError();
}

// One query over a cache of up to this many positions takes k_attn_lds
// (4096 keys: 12.4 against 14.1 us a layer inside a decode token for k_attn;
// the two meet near 8192). Past it, and for a batch of queries on caches of
// their own, a cache at head dimension 128 takes k_attn_m1 (q8, B 16 x 32768
// keys: 248 against 306 us for k_attn), any other k_attn.
constexpr int LDS_MAX_CTX = 8192;

template <int HD, bool F16>
static hipError_t attn_launch(int G, dim3 grid, const AttnArgs &a, hipStream_t s) {
    const int flags = (a.kv_per_batch ? 1 : 0) | (a.append ? 2 : 0) | (a.rope ? 4 : 0);
    const bool lds = grid.z == 1 && a.n_ctx <= LDS_MAX_CTX;
    // Past the LDS kernel, one query per cache at head dimension 128 takes
    // the matrix-core key loop.
    const bool m1 = !lds && HD == 128 && (a.kv_per_batch || grid.z == 1);
    if constexpr (HD == 256) {  // Gemma 3's heads (G 1, 2 or 4): the per-wave kernel
        auto go = [&](auto gc) {
            constexpr int GG = decltype(gc)::value;
            hipLaunchKernelGGL((k_attn<256, GG, F16>), grid, dim3(ATTN_NT), 0, s, (const int8_t *)a.kv.k,
                               (const uint16_t *)a.kv.ks, (const int8_t *)a.kv.v, (const uint16_t *)a.kv.vs, a.n_keys,
                               a.n_ctx, a.HKV, flags, (int)grid.x, a);
        };
        switch (G) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 4: go(std::integral_constant<int, 4>{}); break;
        default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    } else {
#define TS5_ATTN(GG)                                                                                          \
    case GG:                                                                                                  \
        if (lds)                                                                                              \
            hipLaunchKernelGGL((k_attn_lds<HD, GG, F16>), grid, dim3(ATTN_NT), 0, s, (const int8_t *)a.kv.k,  \
                               (const uint16_t *)a.kv.ks, (const int8_t *)a.kv.v, (const uint16_t *)a.kv.vs,  \
                               a.n_keys, a.n_ctx, a.HKV, flags, (int)grid.x, a);                             \
        else                                                                                                  \
            hipLaunchKernelGGL((k_attn<HD, GG, F16>), grid, dim3(ATTN_NT), 0, s, (const int8_t *)a.kv.k,      \
                               (const uint16_t *)a.kv.ks, (const int8_t *)a.kv.v, (const uint16_t *)a.kv.vs,  \
                               a.n_keys, a.n_ctx, a.HKV, flags, (int)grid.x, a);                             \
        break;
    if (m1) return launch_attn_m1(G, F16, grid, a, s);
    switch (G) {
        TS5_ATTN(1)
        TS5_ATTN(2)
        TS5_ATTN(4)
        TS5_ATTN(5)
        TS5_ATTN(7)
        TS5_ATTN(8)
    default: return hipErrorInvalidValue;
    }
#undef TS5_ATTN
    return hipGetLastError();
    }
}

bool attn_mq_fits(int B, int H, int HKV, int HD, int kv_f16, int kv_per_batch) {
    return !kv_f16 && !kv_per_batch && HD == MQ_HD && HKV > 0 && H % HKV == 0 && B >= 2 &&
           B <= ATTN_MAX_NEW && B * (H / HKV) <= MQ_ROWS;
}

bool attn_supported(int H, int HKV, int HD) {
    if (HKV <= 0 || H % HKV) return false;
    const int G = H / HKV;
    if (HD == 256) return G == 1 || G == 2 || G == 4;
    return (HD == 64 || HD == 128) && (G == 1 || G == 2 || G == 4 || G == 5 || G == 7 || G == 8);
}

hipError_t launch_attn(const AttnIO &io, hipStream_t s) {
    // A batch on one cache that appends reads its new keys from LDS: at most ATTN_MAX_NEW.
    if (io.append && !io.kv_per_batch && io.B > ATTN_MAX_NEW) return hipErrorInvalidValue;
    AttnArgs a{};
    a.q = io.q, a.q_stride = io.q_stride, a.bias = io.bias, a.q_norm = io.q_norm, a.k_norm = io.k_norm;
    a.eps = io.eps, a.rope_cs = (const float2 *)io.rope_cs, a.n_rot = io.n_rot, a.neox = io.neox;
    a.rope = io.rope, a.append = io.append, a.kv = io.kv, a.kv_per_batch = io.kv_per_batch, a.n_ctx = io.n_ctx;
    a.H = io.H, a.HKV = io.HKV, a.n_keys = io.n_keys, a.scale = io.scale, a.part = io.part;
    a.counters = io.counters, a.out = io.out;
    a.act_out = (uint8_t *)io.act_out, a.act_stride = io.act_stride, a.win = io.win;
    if (!attn_supported(io.H, io.HKV, io.HD)) return hipErrorInvalidValue;
    const int G = io.H / io.HKV;
    if (!io.win && attn_mq_fits(io.B, io.H, io.HKV, io.HD, io.kv_f16, io.kv_per_batch)) {
        const int flags = (a.append ? 2 : 0) | (a.rope ? 4 : 0);
        hipLaunchKernelGGL(k_attn_mq, dim3(io.n_split, io.HKV), dim3(MQ_NT), 0, s, (const int8_t *)a.kv.k,
                           (const uint16_t *)a.kv.ks, (const int8_t *)a.kv.v, (const uint16_t *)a.kv.vs, a.n_keys,
                           a.n_ctx, a.HKV, flags, io.n_split, G, io.B, a);
        hipLaunchKernelGGL(k_attn_mq_merge, dim3(io.B * G, io.HKV), dim3(MQ_HD), 0, s, a.n_keys, io.n_split, G, io.B,
                           a);
        return hipGetLastError();
    }
    const dim3 grid(io.n_split, io.HKV, io.B);
    if (io.kv_f16)
        return io.HD == 256   ? attn_launch<256, true>(G, grid, a, s)
               : io.HD == 128 ? attn_launch<128, true>(G, grid, a, s)
                              : attn_launch<64, true>(G, grid, a, s);
    return io.HD == 256   ? attn_launch<256, false>(G, grid, a, s)
           : io.HD == 128 ? attn_launch<128, false>(G, grid, a, s)
                          : attn_launch<64, false>(G, grid, a, s);
}

}  // namespace ts5hip
