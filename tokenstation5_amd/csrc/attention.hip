// Decode attention over a q8 KV cache.
//
//  k_rope_kv      per (head, token): bias, optional per-head RMSNorm, RoPE
//                 (engine/src/cpu_backend.cpp:57-68, :198-221), then for K and
//                 V heads the q8 rounding of round_kv (:78-90) written as int8
//                 quants + f16 scales (the split layout of qkv_post.glsl:29-41).
//  k_attn_split   split-K flash decode: per (key slice, KV head) one
//                 workgroup scores its G = H/HKV query heads against 64-key
//                 tiles and keeps an online softmax (attn.glsl:54-162).
//  k_attn_merge   O = sum_s e^(m_s-M) O_s / sum_s e^(m_s-M) l_s
//                 (attn_merge.comp:18-47), written as fp32 and as the Act of
//                 the output projection.
//
// Cache layout per layer: K8/V8 int8 [seq][kv_head][slot][head_dim] and
// Ks/Vs f16 [seq][kv_head][slot][head_dim/32]: one KV head's keys are
// contiguous, 128 + 8 bytes per key at head_dim 128.
#include "common.h"
#include "kernels.h"

namespace ts5hip {

// x0*c - x1*s and x0*s + x1*c with separate roundings, as the reference's
// scalar float code computes them.
__device__ inline void rope_pair(float &x0, float &x1, float c, float s) {
#pragma clang fp contract(off)
    const float a = x0 * c - x1 * s;
    const float b = x0 * s + x1 * c;
    x0 = a;
    x1 = b;
}

__device__ inline float block_sum64(float v) { return wave_sum(v); }

// grid (H + 2*HKV, ntok), 64 threads (one wave): thread i holds values 2i, 2i+1.
__global__ __launch_bounds__(64) void k_rope_kv(const float *__restrict__ qkv, int64_t qkv_stride,
                                                const float *__restrict__ bias, const float *__restrict__ q_norm,
                                                const float *__restrict__ k_norm, float eps,
                                                const float2 *__restrict__ rope_cs, int n_rot, int neox,
                                                const int32_t *__restrict__ pos0p, int H, int HKV, int HD,
                                                int n_ctx, float *__restrict__ q_out, KvLayer kv) {
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
        if (i < n_rot / 2) {
            const int a = neox ? i : 2 * i, b = neox ? i + n_rot / 2 : 2 * i + 1;
            const float2 cs = rope_cs[(int64_t)pos * (n_rot / 2) + i];
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
    // q8: per 32 values sc = f16(amax / 127), q = clamp(rint(v / sc), +-127).
    const int kvh = is_k ? hh - H : hh - H - HKV;
    int8_t *q8 = is_k ? kv.k : kv.v;
    uint16_t *sc8 = is_k ? kv.ks : kv.vs;
    const int64_t slot = (int64_t)kvh * n_ctx + pos;
    if (2 * i < HD) {
        float a0 = v[2 * i], a1 = v[2 * i + 1];
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
        *(uint16_t *)(q8 + slot * HD + 2 * i) = packed;
        if ((i & 15) == 0) sc8[slot * (HD / 32) + (2 * i) / 32] = sh;
    }
}

// ---------------------------------------------------------------------------
// Split-K flash decode. grid (n_split, HKV, B), 256 threads. Query b reads
// keys [0, n_keys[b]) of sequence b (kv_per_batch), or of the one sequence
// keys [0, n_keys[0] + b + 1) (a batch of consecutive positions starting at
// n_keys[0]). Writes the unnormalised partial (sum p*v, m, l) per
// (b, split, head) to part.
// ---------------------------------------------------------------------------
template <int HD, int G>
__global__ __launch_bounds__(256) void k_attn_split(const float *__restrict__ q, KvLayer kv, int kv_per_batch,
                                                    const int32_t *__restrict__ n_keys, int H, int HKV, int n_ctx,
                                                    float scale, float *__restrict__ part) {
    constexpr int TILE = 64, NQ = HD / 4, NPAIR = G * HD / 2, PPT = (NPAIR + 255) / 256;
    __shared__ float q_s[G][HD];
    __shared__ float p_s[G][TILE];
    __shared__ float alpha_s[G], m_s[G], l_s[G];
    const int split = blockIdx.x, kvh = blockIdx.y, b = blockIdx.z, n_split = gridDim.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nk = kv_per_batch ? n_keys[b] : n_keys[0] + b + 1;
    int chunk = (nk + n_split - 1) / n_split;
    chunk = (chunk + TILE - 1) / TILE * TILE;
    const int p0 = split * chunk, p1 = min(nk, p0 + chunk);
    const int seq = kv_per_batch ? b : 0;
    const int64_t head_base = ((int64_t)seq * HKV + kvh) * n_ctx;  // slot index of key 0
    const float *qb = q + ((int64_t)b * H + (int64_t)kvh * G) * HD;
    for (int j = tid; j < G * HD; j += 256) q_s[j / HD][j % HD] = qb[j];
    if (tid < G) {
        m_s[tid] = -INFINITY;
        l_s[tid] = 0.f;
    }
    float o[PPT][2];
#pragma unroll
    for (int k = 0; k < PPT; k++) o[k][0] = o[k][1] = 0.f;
    __syncthreads();

    for (int t0 = p0; t0 < p1; t0 += TILE) {
        // Scores: 4 lanes per key, NQ dims each.
        {
            const int kk = tid >> 2, qq = tid & 3, p = t0 + kk;
            float acc[G];
#pragma unroll
            for (int g = 0; g < G; g++) acc[g] = 0.f;
            if (p < p1) {
                const int8_t *kp = kv.k + (head_base + p) * HD + qq * NQ;
                const float ks = h2f(kv.ks[(head_base + p) * (HD / 32) + (qq * NQ) / 32]);
#pragma unroll
                for (int c = 0; c < NQ / 16; c++) {
                    const uint4 w = *(const uint4 *)(kp + 16 * c);
                    const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const float kf = (float)(int8_t)((ws[e >> 2] >> (8 * (e & 3))) & 0xff) * ks;
                        const int d = qq * NQ + 16 * c + e;
#pragma unroll
                        for (int g = 0; g < G; g++) acc[g] += q_s[g][d] * kf;
                    }
                }
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                acc[g] += __shfl_xor(acc[g], 1, WAVE);
                acc[g] += __shfl_xor(acc[g], 2, WAVE);
            }
            if (qq == 0) {
#pragma unroll
                for (int g = 0; g < G; g++) p_s[g][kk] = p < p1 ? acc[g] * scale : -INFINITY;
            }
        }
        __syncthreads();
        // Online softmax per head: wave w takes heads w, w+4.
        for (int g = wave; g < G; g += 4) {
            const float s = p_s[g][lane];
            const float mt = wave_max(s);
            const float mo = m_s[g];
            const float mn = fmaxf(mo, mt);
            const float p = s == -INFINITY ? 0.f : expf(s - mn);
            const float ls = wave_sum(p);
            p_s[g][lane] = p;
            if (lane == 0) {
                const float al = mo == -INFINITY ? 0.f : expf(mo - mn);
                alpha_s[g] = al;
                m_s[g] = mn;
                l_s[g] = l_s[g] * al + ls;
            }
        }
        __syncthreads();
        // o = o * alpha + sum_k p_k * v_k.
        const int nt = min(TILE, p1 - t0);
#pragma unroll
        for (int k = 0; k < PPT; k++) {
            const int pp = tid + 256 * k;
            if (pp < NPAIR) {
                const int g = (2 * pp) / HD, d = (2 * pp) % HD;
                const float al = alpha_s[g];
                float o0 = o[k][0] * al, o1 = o[k][1] * al;
                const int8_t *vp = kv.v + (head_base + t0) * HD + d;
                const uint16_t *vsp = kv.vs + (head_base + t0) * (HD / 32) + d / 32;
                for (int kk = 0; kk < nt; kk++) {
                    const uint16_t v2 = *(const uint16_t *)(vp + (int64_t)kk * HD);
                    const float w = p_s[g][kk] * h2f(vsp[(int64_t)kk * (HD / 32)]);
                    o0 += w * (float)(int8_t)(v2 & 0xff);
                    o1 += w * (float)(int8_t)(v2 >> 8);
                }
                o[k][0] = o0;
                o[k][1] = o1;
            }
        }
        __syncthreads();
    }
    // Partial record per head: [HD values][m][l].
    float *pb = part + (((int64_t)b * n_split + split) * H + (int64_t)kvh * G) * (HD + 2);
#pragma unroll
    for (int k = 0; k < PPT; k++) {
        const int pp = tid + 256 * k;
        if (pp < NPAIR) {
            const int g = (2 * pp) / HD, d = (2 * pp) % HD;
            pb[g * (HD + 2) + d] = o[k][0];
            pb[g * (HD + 2) + d + 1] = o[k][1];
        }
    }
    if (tid < G) {
        pb[tid * (HD + 2) + HD] = m_s[tid];
        pb[tid * (HD + 2) + HD + 1] = l_s[tid];
    }
}

// grid (H, B), HD threads.
__global__ __launch_bounds__(128) void k_attn_merge(const float *__restrict__ part, int n_split, int H, int HD,
                                                    float *__restrict__ out, uint8_t *__restrict__ act) {
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    const float *pb = part + ((int64_t)b * n_split * H + h) * (HD + 2);
    const int64_t stride = (int64_t)H * (HD + 2);
    float M = -INFINITY;
    for (int s = 0; s < n_split; s++) M = fmaxf(M, pb[s * stride + HD]);
    float L = 0.f, acc = 0.f;
    for (int s = 0; s < n_split; s++) {
        const float m = pb[s * stride + HD];
        const float w = m == -INFINITY ? 0.f : expf(m - M);
        L += w * pb[s * stride + HD + 1];
        acc += w * pb[s * stride + d];
    }
    const float v = acc / L;
    const int64_t n = (int64_t)H * HD;
    if (out) out[(int64_t)b * n + (int64_t)h * HD + d] = v;
    if (act) quant32(v, d & 31, act_view(act + (int64_t)b * act_bytes(n), n), ((int64_t)h * HD + d) / 32);
}

// K (which 0) or V (1) at positions [pos0, pos0 + n) dequantized to fp32
// [n][HKV * HD] (engine/src/cpu_backend.cpp:95-97's row layout).
__global__ void k_kv_read(KvLayer kv, int which, int HKV, int HD, int n_ctx, int pos0, int n, float *__restrict__ out) {
    const int64_t total = (int64_t)n * HKV * HD;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
        const int p = (int)(e / (HKV * HD)), h = (int)(e / HD % HKV), d = (int)(e % HD);
        const int64_t slot = (int64_t)h * n_ctx + pos0 + p;
        const int8_t q = (which ? kv.v : kv.k)[slot * HD + d];
        out[e] = (float)q * h2f((which ? kv.vs : kv.ks)[slot * (HD / 32) + d / 32]);
    }
}

// ---------------------------------------------------------------------------
hipError_t launch_kv_read(KvLayer kv, int which, int HKV, int HD, int n_ctx, int pos0, int n, float *out, hipStream_t s) {
    hipLaunchKernelGGL(k_kv_read, dim3(256), dim3(256), 0, s, kv, which, HKV, HD, n_ctx, pos0, n, out);
    return hipGetLastError();
}

hipError_t launch_rope_kv(const float *qkv, int64_t qkv_stride, const float *bias, const float *q_norm,
                          const float *k_norm, float eps, const float *rope_cs, int n_rot, int neox,
                          const int32_t *pos0, int H, int HKV, int HD, int n_ctx, int ntok, float *q_out, KvLayer kv,
                          hipStream_t s) {
    hipLaunchKernelGGL(k_rope_kv, dim3(H + 2 * HKV, ntok), dim3(64), 0, s, qkv, qkv_stride, bias, q_norm, k_norm,
                       eps, (const float2 *)rope_cs, n_rot, neox, pos0, H, HKV, HD, n_ctx, q_out, kv);
    return hipGetLastError();
}

template <int HD>
static hipError_t split_launch(int G, dim3 grid, const float *q, KvLayer kv, int kv_per_batch, const int32_t *n_keys,
                               int H, int HKV, int n_ctx, float scale, float *part, hipStream_t s) {
#define TS5_SPLIT(GG)                                                                                             \
    case GG:                                                                                                      \
        hipLaunchKernelGGL((k_attn_split<HD, GG>), grid, dim3(256), 0, s, q, kv, kv_per_batch, n_keys, H, HKV, \
                           n_ctx, scale, part);                                                                   \
        break;
    switch (G) {
        TS5_SPLIT(1)
        TS5_SPLIT(2)
        TS5_SPLIT(4)
        TS5_SPLIT(5)
        TS5_SPLIT(7)
        TS5_SPLIT(8)
    default: return hipErrorInvalidValue;
    }
#undef TS5_SPLIT
    return hipGetLastError();
}

bool attn_supported(int H, int HKV, int HD) {
    if (HKV <= 0 || H % HKV) return false;
    const int G = H / HKV;
    return (HD == 64 || HD == 128) && (G == 1 || G == 2 || G == 4 || G == 5 || G == 7 || G == 8);
}

hipError_t launch_attn_decode(const float *q, KvLayer kv, int kv_per_batch, const int32_t *n_keys, int B, int H,
                              int HKV, int HD, int n_ctx, int n_split, float scale, float *part, float *out, void *act,
                              hipStream_t s) {
    const dim3 grid(n_split, HKV, B);
    hipError_t e = HD == 128 ? split_launch<128>(H / HKV, grid, q, kv, kv_per_batch, n_keys, H, HKV, n_ctx, scale,
                                                 part, s)
                             : split_launch<64>(H / HKV, grid, q, kv, kv_per_batch, n_keys, H, HKV, n_ctx, scale,
                                                part, s);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_merge, dim3(H, B), dim3(HD), 0, s, part, n_split, H, HD, out, (uint8_t *)act);
    return hipGetLastError();
}

}  // namespace ts5hip
