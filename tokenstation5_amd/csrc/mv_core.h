// Device core of the one-token k-quant matvec kernels (matvec.hip).
//
// The reference computes y[r] = sum_i deq(W[r,i]) * x[i] with fp64
// accumulation (engine/src/cpu_backend.cpp:18-37); its GPU path reads 8
// lanes per Q4_K super-block with 16-byte loads (mv16_q4_k.glsl:64-113).
// Here:
//  * A workgroup first turns the fp32 input (rms-normalised when a norm
//    weight is given, engine/src/cpu_backend.cpp:48-53) into the quantized
//    activation of common.h in LDS: X = 65536*hi + 256*mid + lo per value
//    (23 significant bits), a scale per 32. The weights are the only HBM
//    stream; the input is read from L2.
//  * Weights stay packed in registers. A lane takes whole 32-value
//    sub-blocks, multiplies raw quants with the activation's three int8
//    planes on v_dot4_i32_i8 (exact int32) and applies the block scales once
//    per sub-block in fp32:
//      Q4_K: y += d*sc*(xs*sum q*X) - dmin*m*(sum x)     (quants.cpp:140-157)
//      Q6_K: y += d*sc*xs*(sum q*X - 32*sum X)           (quants.cpp:179-202)
//      Q8_0: y += d*xs*(sum q*X)                         (quants.cpp:133-139)
//      Q8SM: y += s*xs*(sum q*X) + m*(sum x)   (Q4_0, Q4_1, Q5_0, Q5_1, Q5_K)
//      F16 / F32: y += xs*(sum w*X), w the fp32 value, X exact in fp32
//      (|X| < 2^22), products and sums in fp32 (quants.cpp:78-82)
//  * Persistent row groups: a workgroup walks its groups (R rows per wave)
//    as a flat sequence of steps (one 64-lane sweep of 64/LPB blocks each)
//    and always has the next step's weight loads in flight while it computes
//    the current one. The first step's loads are issued before the
//    activation is built. Rows of many blocks (the down projection) are
//    split between the workgroup's waves, whose sums meet in LDS. Every
//    weight byte is read once.
// Bandwidth-bound: no MFMA.
#pragma once
#include <climits>

#include "common.h"

namespace ts5hip {

struct WPtr {
    const uint8_t *body;     // blocks (Q4_K: whole blocks; Q6_K/Q8_0/Q8SM: bodies)
    const uint16_t *dscale;  // f16 block scales of Q6_K / Q8_0
    const float2 *sm;        // (scale, min) pairs of Q8SM
};

__device__ inline WPtr wptr(uint32_t t, const void *w, int64_t nblocks) {
    WPtr p;
    p.body = (const uint8_t *)w;
    p.dscale = (t == T_Q6_K || t == T_Q8_0) ? (const uint16_t *)(p.body + split_scale_offset(t, nblocks)) : nullptr;
    p.sm = t == T_Q8SM ? (const float2 *)(p.body + split_scale_offset(t, nblocks)) : nullptr;
    return p;
}

__device__ inline uint4 ld16(const void *p) { return *(const uint4 *)p; }

// ---------------------------------------------------------------------------
// Formats. Each lane owns `sub` (0..LPB-1) of every block it visits; a wave
// covers BPI = 64 / LPB consecutive blocks of a row per step.
// ---------------------------------------------------------------------------

// Q4_K: 4 lanes per block, lane `sub` = nibble group g: sub-blocks 2g (low
// nibbles) and 2g+1 (high nibbles), 64 values.
struct Q4K {
    static constexpr int LPB = 4, VALUES = 256;  // lanes per block, values per block
    static constexpr int LOADS = 3;              // vector memory loads per load_w
    struct X {
        uint32_t p[3][2][8];  // [plane hi, mid, lo][sub-block 2 sub, 2 sub + 1][dword]
        float s0, s1, u0, u1;  // the two sub-blocks' scales and sums
    };
    struct W {
        uint4 hdr, qa, qb;
    };
    __device__ static X load_x(const CAct &x, int b, int sub) {
        X r;
        const int base = b * 256 + 64 * sub;
        const int8_t *plane[3] = {x.hi, x.mid, x.lo};
#pragma unroll
        for (int P = 0; P < 3; P++) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const uint4 v = ld16(plane[P] + base + 16 * k);
                uint32_t *d = &r.p[P][k >> 1][4 * (k & 1)];
                d[0] = v.x, d[1] = v.y, d[2] = v.z, d[3] = v.w;
            }
        }
        const int s = b * 8 + 2 * sub;
        r.s0 = x.scale[s];
        r.s1 = x.scale[s + 1];
        r.u0 = x.sum[s];
        r.u1 = x.sum[s + 1];
        return r;
    }
    __device__ static W load_w(const WPtr &w, int64_t row, int nb, int b, int sub) {
        const uint8_t *blk = w.body + ((size_t)row * nb + b) * Q4K_BYTES;
        W r;
        r.hdr = ld16(blk);
        r.qa = ld16(blk + 16 + 32 * sub);
        r.qb = ld16(blk + 32 + 32 * sub);
        return r;
    }
    __device__ static float dot(const W &w, const X &x, int sub) {
        const uint32_t q[8] = {w.qa.x, w.qa.y, w.qa.z, w.qa.w, w.qb.x, w.qb.y, w.qb.z, w.qb.w};
        int a[3][2] = {{0, 0}, {0, 0}, {0, 0}};
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int lo = (int)(q[k] & 0x0F0F0F0Fu), hi = (int)((q[k] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
            for (int P = 0; P < 3; P++) {
                a[P][0] = dot4(lo, (int)x.p[P][0][k], a[P][0]);
                a[P][1] = dot4(hi, (int)x.p[P][1][k], a[P][1]);
            }
        }
        // sum q X per sub-block, exact in int32: |.| <= 32 * 15 * (64 * 65536 +
        // 128 * 256 + 128) = 2,029,056,000 < 2^31.
        const int v0 = a[0][0] * 65536 + a[1][0] * 256 + a[2][0];
        const int v1 = a[0][1] * 65536 + a[1][1] * 256 + a[2][1];
        int sc0, m0, sc1, m1;
        kq_scale_min_pair(sub, w.hdr.y, w.hdr.z, w.hdr.w, sc0, m0, sc1, m1);
        const float d = h2f(w.hdr.x & 0xffff), dmin = h2f(w.hdr.x >> 16);
        const float p = (float)sc0 * x.s0 * (float)v0 + (float)sc1 * x.s1 * (float)v1;
        return d * p - dmin * ((float)m0 * x.u0 + (float)m1 * x.u1);
    }
};

// Q6_K: 4 lanes per block, lane `sub` = (half h = sub/2, i0 = 16*(sub%2)):
// the four 16-value runs at 128h + 32c + i0 (c = 0..3), 64 values.
struct Q6K {
    static constexpr int LPB = 4, VALUES = 256;
    static constexpr int LOADS = 5;  // vector memory loads per load_w
    struct X {
        uint32_t p[3][4][4];  // [plane][run c][dword]
        float s[4];
        int is[4];
    };
    struct W {
        uint4 qla, qlb, qh, sc;
        float d;
    };
    __device__ static X load_x(const CAct &x, int b, int sub) {
        X r;
        const int h = sub >> 1, i0 = (sub & 1) * 16;
        const int8_t *plane[3] = {x.hi, x.mid, x.lo};
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int base = b * 256 + 128 * h + 32 * c + i0;
#pragma unroll
            for (int P = 0; P < 3; P++) {
                const uint4 v = ld16(plane[P] + base);
                r.p[P][c][0] = v.x, r.p[P][c][1] = v.y, r.p[P][c][2] = v.z, r.p[P][c][3] = v.w;
            }
            r.s[c] = x.scale[base / 32];
            r.is[c] = x.isum[base / 16];
        }
        return r;
    }
    __device__ static W load_w(const WPtr &w, int64_t row, int nb, int b, int sub) {
        const size_t blk = (size_t)row * nb + b;
        const uint8_t *body = w.body + blk * Q6K_BODY;
        const int h = sub >> 1, i0 = (sub & 1) * 16;
        W r;
        r.qla = ld16(body + 64 * h + i0);
        r.qlb = ld16(body + 64 * h + 32 + i0);
        r.qh = ld16(body + 128 + 32 * h + i0);
        r.sc = ld16(body + 192);
        r.d = h2f(w.dscale[blk]);
        return r;
    }
    __device__ static float dot(const W &w, const X &x, int sub) {
        const uint32_t qa[4] = {w.qla.x, w.qla.y, w.qla.z, w.qla.w};
        const uint32_t qb[4] = {w.qlb.x, w.qlb.y, w.qlb.z, w.qlb.w};
        const uint32_t qh[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
        int a[3][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t q[4] = {(qa[k] & 0x0F0F0F0Fu) | ((qh[k] << 4) & 0x30303030u),
                                   (qb[k] & 0x0F0F0F0Fu) | ((qh[k] << 2) & 0x30303030u),
                                   ((qa[k] >> 4) & 0x0F0F0F0Fu) | (qh[k] & 0x30303030u),
                                   ((qb[k] >> 4) & 0x0F0F0F0Fu) | ((qh[k] >> 2) & 0x30303030u)};
#pragma unroll
            for (int c = 0; c < 4; c++)
#pragma unroll
                for (int P = 0; P < 3; P++) a[P][c] = dot4((int)q[c], (int)x.p[P][c][k], a[P][c]);
        }
        // Run c's scale is byte 8h + sub%2 + 2c of the 16: dword 2h (c < 2)
        // or 2h + 1 (c >= 2), byte sub%2 + 2(c%2).
        const uint32_t s01 = (sub >> 1) ? w.sc.z : w.sc.x, s23 = (sub >> 1) ? w.sc.w : w.sc.y;
        const int sh = 8 * (sub & 1);
        float p = 0.f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint32_t word = c < 2 ? s01 : s23;
            const int sc = (int)(int8_t)((word >> (sh + 16 * (c & 1))) & 0xff);
            // sum (q - 32) X over the run, exact in 64 bits (q up to 63: the hi
            // plane's term alone can pass 2^31).
            const long long v = (long long)a[0][c] * 65536 + a[1][c] * 256 + a[2][c] - 32ll * x.is[c];
            p += (float)sc * x.s[c] * (float)v;
        }
        return w.d * p;
    }
};

// Q8_0: 2 lanes per 32-value block, 16 values each.
struct Q80 {
    static constexpr int LPB = 2, VALUES = 32;
    static constexpr int LOADS = 2;  // vector memory loads per load_w
    struct X {
        uint4 p[3];  // the planes' 16 bytes
        float s;
    };
    struct W {
        uint4 q;
        float d;
    };
    __device__ static X load_x(const CAct &x, int b, int sub) {
        X r;
        r.p[0] = ld16(x.hi + b * 32 + 16 * sub);
        r.p[1] = ld16(x.mid + b * 32 + 16 * sub);
        r.p[2] = ld16(x.lo + b * 32 + 16 * sub);
        r.s = x.scale[b];
        return r;
    }
    __device__ static W load_w(const WPtr &w, int64_t row, int nb, int b, int sub) {
        const size_t blk = (size_t)row * nb + b;
        W r;
        r.q = ld16(w.body + blk * Q8_BODY + 16 * sub);
        r.d = h2f(w.dscale[blk]);
        return r;
    }
    __device__ static float dot(const W &w, const X &x, int) {
        int a[3] = {0, 0, 0};
#pragma unroll
        for (int P = 0; P < 3; P++) {
            a[P] = dot4((int)w.q.x, (int)x.p[P].x, a[P]);
            a[P] = dot4((int)w.q.y, (int)x.p[P].y, a[P]);
            a[P] = dot4((int)w.q.z, (int)x.p[P].z, a[P]);
            a[P] = dot4((int)w.q.w, (int)x.p[P].w, a[P]);
        }
        const long long v = (long long)a[0] * 65536 + a[1] * 256 + a[2];  // int8 quants: past 2^31 in 64 bits
        return w.d * x.s * (float)v;
    }
};

// Q8SM: Q8_0's lanes and products, and the block's min against the sum of
// its 32 activation values (the unquantized fp32 sum), added by lane 0 of
// the block's pair.
struct Q8M {
    static constexpr int LPB = 2, VALUES = 32;
    static constexpr int LOADS = 2;  // vector memory loads per load_w
    struct X {
        uint4 p[3];
        float s, u;  // scale; the block's sum of x on sub 0, else 0
    };
    struct W {
        uint4 q;
        float2 sm;
    };
    __device__ static X load_x(const CAct &x, int b, int sub) {
        X r;
        r.p[0] = ld16(x.hi + b * 32 + 16 * sub);
        r.p[1] = ld16(x.mid + b * 32 + 16 * sub);
        r.p[2] = ld16(x.lo + b * 32 + 16 * sub);
        r.s = x.scale[b];
        r.u = sub == 0 ? x.sum[b] : 0.f;
        return r;
    }
    __device__ static W load_w(const WPtr &w, int64_t row, int nb, int b, int sub) {
        const size_t blk = (size_t)row * nb + b;
        W r;
        r.q = ld16(w.body + blk * Q8_BODY + 16 * sub);
        r.sm = w.sm[blk];
        return r;
    }
    __device__ static float dot(const W &w, const X &x, int) {
        int a[3] = {0, 0, 0};
#pragma unroll
        for (int P = 0; P < 3; P++) {
            a[P] = dot4((int)w.q.x, (int)x.p[P].x, a[P]);
            a[P] = dot4((int)w.q.y, (int)x.p[P].y, a[P]);
            a[P] = dot4((int)w.q.z, (int)x.p[P].z, a[P]);
            a[P] = dot4((int)w.q.w, (int)x.p[P].w, a[P]);
        }
        const long long v = (long long)a[0] * 65536 + a[1] * 256 + a[2];
        return w.sm.x * x.s * (float)v + w.sm.y * x.u;
    }
};

// F16 and F32 rows, in 32-value blocks (64 / 128 bytes): 16 bytes a lane (8
// halves or 4 floats), against the activation's X = 65536 hi + 256 mid + lo
// rebuilt per value.
__device__ inline float x_value(uint32_t hi, uint32_t mid, uint32_t lo, int k) {
    const int s = 8 * k;
    return (float)((int)(int8_t)(hi >> s) * 65536 + (int)(int8_t)(mid >> s) * 256 + (int)(int8_t)(lo >> s));
}
template <bool HALF>
struct FloatRows {
    static constexpr int VPL = HALF ? 8 : 4;  // values a lane
    static constexpr int LPB = 32 / VPL, VALUES = 32;
    static constexpr int LOADS = 1;
    static constexpr int BYTES = HALF ? 64 : 128;  // a block's bytes
    struct X {
        uint32_t p[3][VPL / 4];  // the lane's values of the three planes
        float s;
    };
    struct W {
        uint4 v;
    };
    __device__ static X load_x(const CAct &x, int b, int sub) {
        X r;
        const int i = b * 32 + VPL * sub;
        const int8_t *plane[3] = {x.hi, x.mid, x.lo};
#pragma unroll
        for (int P = 0; P < 3; P++) {
            if constexpr (HALF) {
                const uint2 v = *(const uint2 *)(plane[P] + i);
                r.p[P][0] = v.x, r.p[P][1] = v.y;
            } else {
                r.p[P][0] = *(const uint32_t *)(plane[P] + i);
            }
        }
        r.s = x.scale[b];
        return r;
    }
    __device__ static W load_w(const WPtr &w, int64_t row, int nb, int b, int sub) {
        return W{ld16(w.body + ((size_t)row * nb + b) * BYTES + 16 * sub)};
    }
    __device__ static float dot(const W &w, const X &x, int) {
        const uint32_t u[4] = {w.v.x, w.v.y, w.v.z, w.v.w};
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < VPL; k++) {
            const float wv = HALF ? h2f((uint16_t)(u[k / 2] >> (16 * (k & 1)))) : __uint_as_float(u[k]);
            acc += wv * x_value(x.p[0][k / 4], x.p[1][k / 4], x.p[2][k / 4], k & 3);
        }
        return x.s * acc;
    }
};
using F16W = FloatRows<true>;
using F32W = FloatRows<false>;

// ---------------------------------------------------------------------------
// The activation prologue: x (n values, optionally rms-normalised by norm_w)
// -> Act in LDS.
// ---------------------------------------------------------------------------
// 1 / sqrt(mean(x^2) + eps) over the n values (1 without norm weights).
template <int NT>
__device__ inline float act_rms(const float *__restrict__ x, const float *__restrict__ norm_w, float eps, int n,
                                float *red) {
    if (!norm_w) return 1.0f;
    float ss = 0.f;
    for (int i = 4 * threadIdx.x; i < n; i += 4 * NT) {
        const float4 v = *(const float4 *)(x + i);
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
    }
    ss = wave_sum(ss);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    ss = 0.f;
#pragma unroll
    for (int w = 0; w < NT / 64; w++) ss += red[w];
    return 1.0f / sqrtf(ss / (float)n + eps);
}

__device__ inline void quant_run(const float (&v)[16], int r, const Act &a) {
    const Run16 q = quant16(v);
    int8_t *plane[3] = {a.hi, a.mid, a.lo};
#pragma unroll
    for (int P = 0; P < 3; P++) *(uint4 *)(plane[P] + 16 * r) = make_uint4(q.pw[P][0], q.pw[P][1], q.pw[P][2], q.pw[P][3]);
    a.isum[r] = q.isum;
    if ((r & 1) == 0) {
        a.scale[r / 2] = q.scale;
        a.sum[r / 2] = q.sum;
    }
}

// The 16-runs r0 + threadIdx.x, r0 + threadIdx.x + NT, ... below r1 of Act a
// (runs 2g and 2g+1 sit in adjacent lanes: NT is a multiple of 64 and r0, r1
// are even, so both are in the loop together).
template <int NT>
__device__ inline void act_runs(const float *__restrict__ x, const float *__restrict__ norm_w, float s, int r0,
                                int r1, const Act &a) {
    for (int r = r0 + threadIdx.x; r < r1; r += NT) {
        float v[16];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 f = *(const float4 *)(x + 16 * r + 4 * k);
            v[4 * k] = f.x, v[4 * k + 1] = f.y, v[4 * k + 2] = f.z, v[4 * k + 3] = f.w;
        }
        if (norm_w) {
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float4 w = *(const float4 *)(norm_w + 16 * r + 4 * k);
                v[4 * k] = v[4 * k] * s * w.x;
                v[4 * k + 1] = v[4 * k + 1] * s * w.y;
                v[4 * k + 2] = v[4 * k + 2] * s * w.z;
                v[4 * k + 3] = v[4 * k + 3] * s * w.w;
            }
        }
        quant_run(v, r, a);
    }
}

template <int NT>
__device__ inline void build_act(const float *__restrict__ x, const float *__restrict__ norm_w, float eps, int n,
                                 const Act &a, float *red) {
    act_runs<NT>(x, norm_w, act_rms<NT>(x, norm_w, eps, n, red), 0, n / 16, a);
    __syncthreads();
}

// The same prologue with its inputs requested up front: thread t's runs
// t, t + NT, ... (at most RUNS) of x, and of the norm weights with NORM, go to
// registers before the weight loads are issued, so they come back first
// (loads complete in order) and the norm's sum and the quantization need no
// second pass over memory.
template <int NT, int RUNS, bool NORM>
struct ActIn {
    float4 x[RUNS][4];
    float4 w[NORM ? RUNS : 1][4];
};
template <int NT, int RUNS, bool NORM>
__device__ inline void act_in_load(ActIn<NT, RUNS, NORM> &in, const float *__restrict__ x,
                                   const float *__restrict__ norm_w, int n) {
    const int nr = n / 16;
#pragma unroll
    for (int k = 0; k < RUNS; k++) {
        const int r = min((int)threadIdx.x + NT * k, nr - 1);  // past the end: a valid run, not used
#pragma unroll
        for (int j = 0; j < 4; j++) {
            in.x[k][j] = *(const float4 *)(x + 16 * r + 4 * j);
            if constexpr (NORM) in.w[k][j] = *(const float4 *)(norm_w + 16 * r + 4 * j);
        }
    }
}
template <int NT, int RUNS, bool NORM>
__device__ inline void act_in_build(const ActIn<NT, RUNS, NORM> &in, float eps, int n, const Act &a, float *red) {
    const int nr = n / 16;
    float s = 1.0f;
    if constexpr (NORM) {
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < RUNS; k++) {
            if ((int)threadIdx.x + NT * k >= nr) continue;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 v = in.x[k][j];
                ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            }
        }
        ss = wave_sum_dpp(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        ss = 0.f;
#pragma unroll
        for (int w = 0; w < NT / 64; w++) ss += red[w];
        s = 1.0f / sqrtf(ss / (float)n + eps);
    }
#pragma unroll
    for (int k = 0; k < RUNS; k++) {
        const int r = (int)threadIdx.x + NT * k;
        if (r >= nr) continue;
        float v[16];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float4 f = in.x[k][j];
            v[4 * j] = f.x, v[4 * j + 1] = f.y, v[4 * j + 2] = f.z, v[4 * j + 3] = f.w;
            if constexpr (NORM) {
                const float4 w = in.w[k][j];
                v[4 * j] = v[4 * j] * s * w.x;
                v[4 * j + 1] = v[4 * j + 1] * s * w.y;
                v[4 * j + 2] = v[4 * j + 2] * s * w.z;
                v[4 * j + 3] = v[4 * j + 3] * s * w.w;
            }
        }
        quant_run(v, r, a);
    }
    __syncthreads();
}

enum { MV_STORE = 0, MV_ADD = 1, MV_GLU = 2, MV_ARGMAX = 3 };

struct MvArgs {
    uint32_t t;
    const void *w, *w2;  // w2: the up projection of MV_GLU
    int64_t nrows;
    int nb, n_in;
    const float *x, *norm_w;
    float eps;
    float *y;
    const float *y_in;  // MV_ADD: y[r] = y_in[r] + W x (y_in may be y)
    // MV_ARGMAX: per-workgroup best (value, row), the last workgroup's counter,
    // and where the winning id goes: out[0], and seq[*pos + 1] with ++*pos
    // when seq is given.
    float *best_v;
    int *best_i, *counter;
    int32_t *out, *seq, *pos;
    // A persistent grid's groups: with n1 > 0, the first nfirst workgroups
    // (dispatched first, one a CU) take groups [0, n1) in turn and the others
    // [n1, ngroups); else workgroup wg takes wg, wg + nwg, ...
    int nfirst, n1;
    int gelu;  // MV_GLU: GELU (tanh form) for SiLU
};

// The arguments only some modes need, passed after the others.
struct MvTail {
    uint32_t t;
    int nb, nfirst, n1;
    const float *y_in;
    float *best_v;
    int *best_i, *counter;
    int32_t *out, *seq, *pos;
    int gelu;
};

// The row-packed matvec kernels (mv_run's BR = 4: Q4_K, one row a slot, 4
// waves), in matvec_packed.hip: mode MV_STORE / MV_ADD / MV_GLU, the
// prologue's runs per thread (0: two-pass), norm fused.
hipError_t launch_mv_packed(int mode, int runs, bool norm, dim3 g, dim3 b, size_t lds, hipStream_t s, const void *w,
                            const void *w2, const float *x, const float *norm_w, float *y, int nrows, int n_in,
                            int nwg, float eps, const MvTail &tail);

template <class F, int R>
__device__ inline void load_rows(const WPtr &w, int64_t row0, int64_t nrows, int nb, int b, int bmax, int sub,
                                 typename F::W (&wf)[R]) {
    const int bb = min(b, bmax);  // lanes past the split's end re-read its last block (in bounds), not used
#pragma unroll
    for (int r = 0; r < R; r++) wf[r] = F::load_w(w, min(row0 + r, nrows - 1), nb, bb, sub);
}


// (v, i) across the wave: larger value, then lower index.
__device__ inline void best_pick_wave(float &v, int &i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float w = __shfl_xor(v, o, WAVE);
        const int j = __shfl_xor(i, o, WAVE);
        if (w > v || (w == v && j < i)) v = w, i = j;
    }
}

// The workgroup `wg` of `nwg` computes its row groups of a. Its WAVES waves
// are KS splits of WAVES / KS row waves: row wave rw takes rows rw*R ..
// rw*R + R-1 of each group, split ks the blocks ks*nbk .. ks*nbk + nbk-1 of
// those rows (nbk = ceil(nb / KS)); the splits' sums meet in LDS and the
// first split finishes the rows, adding them in split order. before_act()
// runs after the first weight loads are issued and before the activation is
// built. lds: act_bytes(a.n_in) bytes; red: NT/64 floats. MV_ARGMAX returns
// this workgroup's best (value, row) in best_v / best_i (every thread).
// BR (0: a step sweeps BPI blocks of each of the wave's R rows) = 4: a step
// sweeps 4 blocks of 4 times as many rows, each 16-lane row of the wave on
// its own matrix row, so rows whose block count is a multiple of 4 but not
// of BPI (5120 wide: 20 Q4_K blocks) fill every step instead of leaving most
// of their last one empty; one split, no pick.
template <class F, int R, int WAVES, int KS, int MODE, int RUNS, bool NORM, int BR = 0, class Hook>
__device__ inline void mv_run(const MvArgs &a, int wg, int nwg, uint8_t *lds, float *red, Hook before_act,
                              float &best_v, int &best_i) {
    static_assert(WAVES % KS == 0, "splits of whole row waves");
    constexpr int NT = WAVES * WAVE, BPI = WAVE / F::LPB, NW = MODE == MV_GLU ? 2 : 1, RW = WAVES / KS;
    constexpr int BS = BR ? BR : BPI, LR = BPI / BS;  // blocks of a row a step; rows a slot's lanes span
    static_assert(BR == 0 || (BR * F::LPB == 16 && KS == 1 && MODE != MV_ARGMAX && R <= 16),
                  "row-packed steps: 16-lane rows, one split, no pick");
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, bsub = lane / F::LPB, sub = lane % F::LPB;
    const int rw = wave % RW, ks = wave / RW;
    const int64_t rpg = (int64_t)R * LR * RW;
    const int64_t ngroups = (a.nrows + rpg - 1) / rpg;
    const int nbk = KS == 1 ? a.nb : (a.nb + KS - 1) / KS;
    const int spg = (nbk + BS - 1) / BS;  // steps per row group
    const int kb0 = ks * nbk, kb1 = min(a.nb, kb0 + nbk);
    const int64_t nblocks = (int64_t)a.nb * a.nrows;
    const WPtr w1 = wptr(a.t, a.w, nblocks), w2 = wptr(a.t, MODE == MV_GLU ? a.w2 : a.w, nblocks);
    best_v = -INFINITY;
    best_i = INT_MAX;
    // The splits' row sums, double-buffered by group parity: the first split
    // reads buffer p after the barrier of its group, and a split writes p
    // again only after the next group's barrier, which that read precedes.
    __shared__ float kpart[KS > 1 ? 2 : 1][KS][RW][NW][R];

    // Every argument the prologue and the first loads need, fetched together
    // (the compiler would fetch each where first used: a round trip apiece).
    asm volatile("" ::"s"(a.w), "s"(a.w2), "s"(a.x), "s"(a.norm_w), "s"(a.y), "s"(a.nrows), "s"(a.nb), "s"(a.n_in),
                 "s"(a.eps), "s"(nwg));
    // This workgroup's groups: gbeg, gbeg + gstr, ... below gend.
    int64_t gbeg = wg, gstr = nwg, gend = ngroups;
    if (a.n1 > 0) {
        if (wg < a.nfirst) gstr = a.nfirst, gend = a.n1;
        else gbeg = a.n1 + (wg - a.nfirst), gstr = nwg - a.nfirst;
    }
    int64_t g = gbeg;
    int it = 0;
    ActIn<NT, RUNS ? RUNS : 1, NORM> ain;
    if constexpr (RUNS > 0) act_in_load<NT, RUNS, NORM>(ain, a.x, a.norm_w, a.n_in);
    typename F::W cur[NW][R], nxt[NW][R];
    // The weights of step `i` of group `gi` into `buf`.
    auto issue = [&](int64_t gi, int i, typename F::W (&buf)[NW][R]) {
        if constexpr (BR == 0) {
            const int64_t row0 = gi * rpg + (int64_t)rw * R;
            load_rows<F, R>(w1, row0, a.nrows, a.nb, kb0 + i * BPI + bsub, kb1 - 1, sub, buf[0]);
            if (MODE == MV_GLU) load_rows<F, R>(w2, row0, a.nrows, a.nb, kb0 + i * BPI + bsub, kb1 - 1, sub, buf[NW - 1]);
        } else {  // slot r: row row0 + r LR + lrow (clamped), block kb0 + i BS + lblk (clamped)
            const int lrow = bsub / BS, lblk = bsub % BS;
            const int64_t row0 = gi * rpg + (int64_t)rw * R * LR + lrow;
            const int bb = min(kb0 + i * BS + lblk, kb1 - 1);
#pragma unroll
            for (int r = 0; r < R; r++) {
                const int64_t row = min(row0 + (int64_t)r * LR, a.nrows - 1);
                buf[0][r] = F::load_w(w1, row, a.nb, bb, sub);
                if (MODE == MV_GLU) buf[NW - 1][r] = F::load_w(w2, row, a.nb, bb, sub);
            }
        }
    };
    // Unconditional (rows are clamped; every workgroup has gbeg < gend), so no
    // branch makes the compiler's waits for the activation cover these.
    // (Issuing the second step here as well, before the activation is built,
    // measured slower: the input's loads then return later.)
    issue(g, 0, cur);
    before_act();
    const Act xa = act_view(lds, a.n_in);
    if constexpr (RUNS > 0) act_in_build<NT, RUNS, NORM>(ain, a.eps, a.n_in, xa, red);
    else if (g < gend) build_act<NT>(a.x, a.norm_w, a.eps, a.n_in, xa, red);
    const CAct x{xa.hi, xa.mid, xa.lo, xa.scale, xa.sum, xa.isum};
    // The input runs (older than the first step's weights) are all in; said
    // explicitly, so that the compiler's count does not carry those of
    // threads that had no run into the loop as still open (it then waited
    // for most of a step's loads before issuing the next step's).
    wait_vmcnt<F::LOADS * R * NW>();

    float acc[NW][R];
#pragma unroll
    for (int k = 0; k < NW; k++)
#pragma unroll
        for (int r = 0; r < R; r++) acc[k][r] = 0.f;
    int par = 0;
    // Step `it` of group g on the weights in cb; at the group's last step, the
    // rows' results.
    auto compute = [&](const typename F::W (&cb)[NW][R]) {
        // Branch-free: lanes past the split's end compute on its last block
        // (loaded clamped) and add nothing, so no path skips the arithmetic
        // whose waits the compiler must then assume still open.
        int b;
        if constexpr (BR == 0) b = kb0 + it * BPI + bsub;
        else b = kb0 + it * BS + bsub % BS;
        const bool valid = b < kb1;
        const typename F::X xf = F::load_x(x, min(b, kb1 - 1), sub);
#pragma unroll
        for (int k = 0; k < NW; k++)
#pragma unroll
            for (int r = 0; r < R; r++) {
                const float d = F::dot(cb[k][r], xf, sub);
                acc[k][r] += valid ? d : 0.f;
            }
        if (it != spg - 1) return;
        if constexpr (BR == 0) {
#pragma unroll
            for (int k = 0; k < NW; k++)
#pragma unroll
                for (int r = 0; r < R; r++) acc[k][r] = wave_sum_dpp(acc[k][r]);
        } else {
#pragma unroll
            for (int k = 0; k < NW; k++)
#pragma unroll
                for (int r = 0; r < R; r++) acc[k][r] = row_sum_dpp(acc[k][r]);
        }
        if constexpr (KS > 1) {
            if (lane == 0)
#pragma unroll
                for (int k = 0; k < NW; k++)
#pragma unroll
                    for (int r = 0; r < R; r++) kpart[par][ks][rw][k][r] = acc[k][r];
            __syncthreads();
            if (ks == 0)
#pragma unroll
                for (int k = 0; k < NW; k++)
#pragma unroll
                    for (int r = 0; r < R; r++) {
                        float v = kpart[par][0][rw][k][r];
#pragma unroll
                        for (int j = 1; j < KS; j++) v += kpart[par][j][rw][k][r];
                        acc[k][r] = v;
                    }
            par ^= 1;
        }
        if constexpr (BR != 0) {  // slot r: lane r of each 16-lane row, row row0 + r LR + that row's index
            const int wl = lane & 15;
            const int64_t row0 = g * rpg + (int64_t)rw * R * LR + bsub / BS;
            if (wl < R && row0 + (int64_t)wl * LR < a.nrows) {
                float v = acc[0][0], u = acc[NW - 1][0];
#pragma unroll
                for (int r = 1; r < R; r++)
                    if (wl == r) v = acc[0][r], u = acc[NW - 1][r];
                const int64_t row = row0 + (int64_t)wl * LR;
                if (MODE == MV_ADD) st_dev(a.y + row, a.y_in[row] + v);
                else if (MODE == MV_GLU) st_dev(a.y + row, glu_act(v, u, a.gelu));
                else st_dev(a.y + row, v);
            }
#pragma unroll
            for (int k = 0; k < NW; k++)
#pragma unroll
                for (int r = 0; r < R; r++) acc[k][r] = 0.f;
            return;
        }
        const int64_t row0 = g * rpg + (int64_t)rw * R;
        if (ks == 0 && lane < R && row0 + lane < a.nrows) {
            float v = acc[0][0], u = acc[NW - 1][0];
#pragma unroll
            for (int r = 1; r < R; r++)
                if (lane == r) v = acc[0][r], u = acc[NW - 1][r];
            const int64_t row = row0 + lane;
            if (MODE == MV_ADD) {
                st_dev(a.y + row, a.y_in[row] + v);
            } else if (MODE == MV_GLU) {
                st_dev(a.y + row, glu_act(v, u, a.gelu));
            } else {
                st_dev(a.y + row, v);
                if (MODE == MV_ARGMAX && (v > best_v || (v == best_v && row < best_i))) best_v = v, best_i = (int)row;
            }
        }
#pragma unroll
        for (int k = 0; k < NW; k++)
#pragma unroll
            for (int r = 0; r < R; r++) acc[k][r] = 0.f;
    };
    // The steps of this workgroup (its groups wg, wg + nwg, ... times spg) run
    // through the two register buffers in turn: the next step's loads are
    // issued, unconditionally, right before this step's arithmetic in the
    // same block, so the compiler's wait for this step's weights leaves the
    // next step's in flight. (Loads issued under a branch that joins before
    // the arithmetic made it wait for all of them, vmcnt(0), and a copy from
    // one buffer to the other waits for the copied loads.) Only the last step
    // is computed with nothing behind it.
    const int64_t nsteps = (gend - gbeg + gstr - 1) / gstr * spg;
    auto issue_next = [&](typename F::W (&buf)[NW][R]) {  // the step after (g, it)
        int64_t gn = g;
        int itn = it + 1;
        if (itn == spg) itn = 0, gn = g + gstr;
        issue(gn, itn, buf);
    };
    auto advance = [&]() {
        if (++it == spg) it = 0, g += gstr;
    };
    for (int64_t s = 0;; s += 2) {
        if (s + 1 >= nsteps) {
            compute(cur);
            break;
        }
        issue_next(nxt);
        compute(cur);
        advance();
        if (s + 2 >= nsteps) {
            compute(nxt);
            break;
        }
        issue_next(cur);
        compute(nxt);
        advance();
    }
    if (MODE == MV_ARGMAX) {
        // The first maximum wins (std::max_element): larger value, then lower row.
        best_pick_wave(best_v, best_i);
        __syncthreads();
        if (lane == 0) red[wave] = best_v, red[WAVES + wave] = __int_as_float(best_i);
        __syncthreads();
        for (int k = 0; k < WAVES; k++) {
            const float v = red[k];
            const int i = __float_as_int(red[WAVES + k]);
            if (v > best_v || (v == best_v && i < best_i)) best_v = v, best_i = i;
        }
        __syncthreads();
    }
}

}  // namespace ts5hip
