// Weight formats: GGUF -> HBM layout (repack), random-init weights generated
// in HBM, and exact unpack to fp32 (dequantize, embedding lookup).
//
// Unpack follows engine/src/quants.cpp:74-205 operation for operation; each
// product there is exact in fp32 (Q4_K d*sc*q and dmin*m need <= 21 bits,
// Q6_K d*sc*q <= 24 bits, Q8_0 q*d <= 19 bits), so the result is bit-exact
// whether or not the compiler contracts to FMA.
#include "common.h"
#include "kernels.h"

namespace ts5hip {

__global__ void k_dequant(uint32_t t, const uint8_t *__restrict__ w, int64_t ne0, int64_t rows, float *__restrict__ y) {
    const int bv = block_values(t);
    const int nb = (int)(ne0 / bv);
    const int64_t nblocks = (int64_t)nb * rows;
    const int64_t n = ne0 * rows;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = e / ne0, i = e % ne0;
        y[e] = unpack_value(t, w, nblocks, row, t == T_F32 || t == T_F16 ? (int)ne0 : nb, i);
    }
}

// Embedding lookup (engine/src/cpu_backend.cpp:124-134): x[t] = row
// ids[p0 + t], p0 = *pos (0 when pos is null).
__global__ void k_embed(uint32_t t, const uint8_t *__restrict__ w, int64_t ne0, int64_t n_rows,
                        const int32_t *__restrict__ ids, const int32_t *__restrict__ pos, float *__restrict__ x,
                        float scale) {
    const int bv = block_values(t);
    const int nb = (int)(ne0 / bv);
    int64_t row = ids[(pos ? pos[0] : 0) + (int)blockIdx.x];
    if (row < 0 || row >= n_rows) row = 0;  // ids are checked on the host; never read out of bounds
    float *out = x + (int64_t)blockIdx.x * ne0;
    // One value per thread (grid.y covers the row): every value's loads are
    // independent, so a token costs one memory round trip, not one per value.
    const int64_t i = (int64_t)blockIdx.y * blockDim.x + threadIdx.x;
    if (i >= ne0) return;
    const float v = unpack_value(t, w, (int64_t)nb * n_rows, row, t == T_F32 || t == T_F16 ? (int)ne0 : nb, i);
    out[i] = scale > 0.f ? v * scale : v;  // Gemma 3's sqrt(n_embd) (engine/src/cpu_backend.cpp:132-133)
}

// ---------------------------------------------------------------------------
// Repack: GGUF bytes (already in HBM) -> HBM layout. One thread per block.
// ---------------------------------------------------------------------------
__global__ void k_repack_split(uint32_t t, const uint8_t *__restrict__ src, int64_t nblocks, uint8_t *__restrict__ dst,
                               uint16_t *__restrict__ ds) {
    for (int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; blk < nblocks;
         blk += (int64_t)gridDim.x * blockDim.x) {
        if (t == T_Q6_K) {
            const uint8_t *b = src + blk * 210;
            uint8_t *o = dst + blk * Q6K_BODY;
            for (int i = 0; i < Q6K_BODY; i++) o[i] = b[i];
            ds[blk] = (uint16_t)(b[208] | (b[209] << 8));
        } else {  // Q8_0
            const uint8_t *b = src + blk * 34;
            uint8_t *o = dst + blk * Q8_BODY;
            for (int i = 0; i < Q8_BODY; i++) o[i] = b[2 + i];
            ds[blk] = (uint16_t)(b[0] | (b[1] << 8));
        }
    }
}

// GGUF Q4_0 / Q4_1 / Q5_0 / Q5_1 / Q5_K blocks -> T_Q8SM (common.h): int8
// quants, 32 a block, and (s, m) with value = s * q + m, the reference's
// unpack (engine/src/quants.cpp:89-131, :157-177). One thread per GGUF block
// (a Q5_K block is 8 layout blocks).
__device__ inline float f16_at(const uint8_t *p) { return h2f((uint16_t)(p[0] | (p[1] << 8))); }

__global__ void k_repack_sm(uint32_t t, const uint8_t *__restrict__ src, int64_t nblocks, int8_t *__restrict__ dst,
                            float2 *__restrict__ sm) {
    for (int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; blk < nblocks;
         blk += (int64_t)gridDim.x * blockDim.x) {
        if (t == T_Q5_K) {
            const uint8_t *b = src + blk * 176;
            const float d = f16_at(b), dmin = f16_at(b + 2);
            const uint8_t *sc = b + 4, *qh = b + 16, *ql = b + 48;
            const uint32_t *scw = (const uint32_t *)sc;  // 4-byte aligned: 176 B blocks
            for (int j = 0; j < 8; j++) {
                int s6, m6;
                kq_scale_min(j, scw[0], scw[1], scw[2], s6, m6);
                int8_t *o = dst + (blk * 8 + j) * Q8_BODY;
                const uint8_t *q4 = ql + 32 * (j / 2);
                for (int l = 0; l < 32; l++) {
                    const int lo = j & 1 ? q4[l] >> 4 : q4[l] & 15;
                    o[l] = (int8_t)(lo | (((qh[l] >> j) & 1) << 4));
                }
                sm[blk * 8 + j] = make_float2(d * (float)s6, -(dmin * (float)m6));
            }
            continue;
        }
        const int bytes = gguf_block_bytes(t);
        const uint8_t *b = src + blk * bytes;
        const bool has_min = t == T_Q4_1 || t == T_Q5_1, five = t == T_Q5_0 || t == T_Q5_1;
        const float d = f16_at(b), m = has_min ? f16_at(b + 2) : -0.0f;
        const uint8_t *h = b + (has_min ? 4 : 2);
        const uint32_t qh = five ? (uint32_t)h[0] | (uint32_t)h[1] << 8 | (uint32_t)h[2] << 16 | (uint32_t)h[3] << 24 : 0;
        const uint8_t *qs = h + (five ? 4 : 0);
        const int off = has_min ? 0 : five ? 16 : 8;  // Q4_0: nibble - 8, Q5_0: 5-bit - 16
        int8_t *o = dst + blk * Q8_BODY;
        for (int j = 0; j < 16; j++) {
            const int x0 = (qs[j] & 15) | (int)(((qh >> j) & 1) << 4);
            const int x1 = (qs[j] >> 4) | (int)(((qh >> (j + 16)) & 1) << 4);
            o[j] = (int8_t)(x0 - off);
            o[j + 16] = (int8_t)(x1 - off);
        }
        sm[blk] = make_float2(d, m);
    }
}

// ---------------------------------------------------------------------------
// Random-init weights in HBM (benchmark inputs; no checkpoint is reachable).
// Field distributions of the benchmark configs: uniform quant bytes, uniform
// packed K-quant scale bytes (= uniform 6-bit scales and mins), f16 block
// scales |N(0,1)| * 0.01, fp32 norm weights N(1, 0.02). Counter-based: value
// k of stream (seed, tensor) is a hash of its index, so any launch shape
// gives the same tensor.
// ---------------------------------------------------------------------------
__device__ inline uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ull;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
__device__ inline float unit(uint64_t h) { return ((float)(h >> 40) + 0.5f) * (1.0f / 16777216.0f); }
__device__ inline float normal(uint64_t key) {
    const uint64_t h = mix64(key);
    const float u1 = unit(h), u2 = unit(mix64(h ^ 0x5bd1e995ull));
    return sqrtf(-2.0f * logf(u1)) * cosf(6.28318530718f * u2);
}

// One block of the tensor, written in its HBM layout (split layouts: body
// at dst, f16 scale at ds).
__device__ void synth_block(uint32_t t, uint64_t seed, int centered, uint8_t *__restrict__ dst,
                            uint16_t *__restrict__ ds, int64_t blk) {
    const uint64_t key = mix64(seed) ^ ((uint64_t)blk * 0x100000001b3ull);
    auto word = [&](int k) { return (uint32_t)mix64(key + (uint64_t)k * 0x9e3779b97f4a7c15ull); };
    if (t == T_F32) {
        ((float *)dst)[blk] = 1.0f + 0.02f * normal(key);
    } else if (t == T_F16) {
        ((uint16_t *)dst)[blk] = f2h(normal(key));
    } else if (t == T_Q4_K) {
        uint32_t *o = (uint32_t *)(dst + blk * Q4K_BYTES);
        for (int k = 1; k < 36; k++) o[k] = word(k);
        const float d = fabsf(normal(key ^ 0xd1ull)) * 0.01f;
        if (centered) {
            // dmin = 8 d and min_j = round(7.5 scale_j / 8): each sub-block's
            // values centre near zero.
            const uint16_t dh = f2h(d);
            o[0] = dh | ((uint32_t)f2h(h2f(dh) * 8.0f) << 16);
            uint8_t sc[8], mn[8];
            for (int j = 0; j < 8; j++) {
                sc[j] = (uint8_t)((word(40 + j) >> 7) & 63);
                mn[j] = (uint8_t)rintf(sc[j] * 7.5f / 8.0f);
            }
            uint8_t *s = (uint8_t *)(o + 1);
            for (int j = 0; j < 4; j++) {
                s[j] = sc[j] | ((sc[j + 4] >> 4) << 6);
                s[j + 4] = mn[j] | ((mn[j + 4] >> 4) << 6);
                s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4);
            }
        } else {
            const float dm = fabsf(normal(key ^ 0xd2ull)) * 0.01f;
            o[0] = f2h(d) | ((uint32_t)f2h(dm) << 16);
        }
    } else if (t == T_Q6_K || t == T_Q8_0) {
        const int body = t == T_Q6_K ? Q6K_BODY : Q8_BODY;
        uint32_t *o = (uint32_t *)(dst + blk * body);
        for (int k = 0; k < body / 4; k++) o[k] = word(k);
        ds[blk] = f2h(fabsf(normal(key ^ 0xd1ull)) * 0.01f);
    }
}

__global__ void k_synth(uint32_t t, int64_t nblocks, uint64_t seed, int centered, uint8_t *__restrict__ dst,
                        uint16_t *__restrict__ ds) {
    for (int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; blk < nblocks;
         blk += (int64_t)gridDim.x * blockDim.x)
        synth_block(t, seed, centered, dst, ds, blk);
}

// A synthetic KV cache (benchmark inputs): n values drawn N(0,1), stored as
// the cache keeps them: q8 as round_kv does (engine/src/cpu_backend.cpp:78-90:
// per 32 values sc = f16(amax / 127), q = clamp(rint(v / sc), +-127); values
// at q, scales at sc, one per 32 consecutive values) or f16. One thread per
// 32-value block; value k of the stream is a hash of (seed, k).
__global__ void k_kv_synth(int64_t nblocks, uint64_t seed, int kv_f16, uint8_t *__restrict__ vals,
                           uint16_t *__restrict__ scales) {
    const uint64_t base = mix64(seed ^ 0x6b76ull);
    for (int64_t blk = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; blk < nblocks;
         blk += (int64_t)gridDim.x * blockDim.x) {
        float v[32];
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            v[i] = normal(base + (uint64_t)(blk * 32 + i) * 0x9e3779b97f4a7c15ull);
            amax = fmaxf(amax, fabsf(v[i]));
        }
        if (kv_f16) {
            uint32_t *o = (uint32_t *)(vals + blk * 64);
#pragma unroll
            for (int i = 0; i < 16; i++) o[i] = (uint32_t)f2h(v[2 * i]) | (uint32_t)f2h(v[2 * i + 1]) << 16;
            continue;
        }
        const uint16_t sh = f2h(amax / 127.0f);
        const float sc = h2f(sh);
        uint32_t *o = (uint32_t *)(vals + blk * 32);
#pragma unroll
        for (int w = 0; w < 8; w++) {
            uint32_t word = 0;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int q = sc > 0.f ? (int)fminf(127.f, fmaxf(-127.f, rintf(v[4 * w + b] / sc))) : 0;
                word |= (uint32_t)(q & 0xff) << (8 * b);
            }
            o[w] = word;
        }
        scales[blk] = sh;
    }
}

// ---------------------------------------------------------------------------
// Launchers.
// ---------------------------------------------------------------------------
static int grid_for(int64_t n, int block) {
    int64_t g = (n + block - 1) / block;
    return (int)(g > (1 << 20) ? (1 << 20) : (g < 1 ? 1 : g));
}

hipError_t launch_dequant(uint32_t t, const void *w, int64_t ne0, int64_t rows, float *y, hipStream_t s) {
    hipLaunchKernelGGL(k_dequant, dim3(grid_for(ne0 * rows, 256)), dim3(256), 0, s, t, (const uint8_t *)w, ne0, rows,
                       y);
    return hipGetLastError();
}

hipError_t launch_embed(uint32_t t, const void *w, int64_t ne0, int64_t n_rows, const int32_t *ids, const int32_t *pos,
                        int ntok, float *x, hipStream_t s, float scale) {
    hipLaunchKernelGGL(k_embed, dim3(ntok, (unsigned)((ne0 + 255) / 256)), dim3(256), 0, s, t, (const uint8_t *)w, ne0,
                       n_rows, ids, pos, x, scale);
    return hipGetLastError();
}

hipError_t launch_repack(uint32_t t, int64_t nblocks, const void *gguf, void *body, void *scales, hipStream_t s) {
    if (device_type(t) == T_Q8SM)
        hipLaunchKernelGGL(k_repack_sm, dim3(grid_for(nblocks, 256)), dim3(256), 0, s, t, (const uint8_t *)gguf,
                           nblocks, (int8_t *)body, (float2 *)scales);
    else
        hipLaunchKernelGGL(k_repack_split, dim3(grid_for(nblocks, 256)), dim3(256), 0, s, t, (const uint8_t *)gguf,
                           nblocks, (uint8_t *)body, (uint16_t *)scales);
    return hipGetLastError();
}

hipError_t launch_synth(uint32_t t, int64_t ne0, int64_t nrows, uint64_t seed, int centered, void *body, void *scales,
                        hipStream_t s) {
    const int64_t nb = ne0 / block_values(t) * nrows;
    hipLaunchKernelGGL(k_synth, dim3(grid_for(nb, 256)), dim3(256), 0, s, t, nb, seed, centered, (uint8_t *)body,
                       (uint16_t *)scales);
    return hipGetLastError();
}

hipError_t launch_kv_synth(int64_t n, uint64_t seed, int kv_f16, void *vals, void *scales, hipStream_t s) {
    const int64_t nb = n / 32;
    hipLaunchKernelGGL(k_kv_synth, dim3(grid_for(nb, 256)), dim3(256), 0, s, nb, seed, kv_f16, (uint8_t *)vals,
                       (uint16_t *)scales);
    return hipGetLastError();
}

}  // namespace ts5hip
