// Device core of split-K flash decode over the KV cache (q8, or f16), used
// by the kernels of attention.hip.
#pragma once
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace ts5hip {
constexpr int ATTN_MIN_KEYS = 128;  // the fewest keys a split takes
// Up to this many keys one work item takes them all: merging slices costs
// ~2.3 us (the partials' writes, the count, the merge's read), more than one
// work item spends on 256 keys (decode at 129-256 keys: 8.8 against 9.7 us,
// 32/8 heads of 128; past 256 the LDS kernel's second pass of keys costs
// more than the merge: 12.0 against 9.8 us at 384).
constexpr int ATTN_SINGLE_MAX = 256;
constexpr int ATTN_DEPTH = 2;       // chunks of K and V in flight per wave (attn_slice; 3 and 4 measured slower)

// x0*c - x1*s and x0*s + x1*c with separate roundings, as the reference's
// scalar float code computes them (engine/src/cpu_backend.cpp:63-64).
__device__ inline void rope_pair(float &x0, float &x1, float c, float s) {
#pragma clang fp contract(off)
    const float a = x0 * c - x1 * s;
    const float b = x0 * s + x1 * c;
    x0 = a;
    x1 = b;
}

// ---------------------------------------------------------------------------
// Split-K flash decode with the token's own preparation and the merge fused
// in. grid (n_split, HKV, B), NT threads; query b is at position nk - 1
// and reads keys [0, nk):
//   nk = n_keys[b] (kv_per_batch: B independent caches), or
//   nk = n_keys[0] + b + 1 (one cache, a batch of consecutive positions).
// 1. The G query heads of this KV head: q (+ bias, per-head norm, RoPE
//    when `rope`) -> LDS.
// 2. `append`: the batch's new keys (one cache: positions n_keys[0] ..
//    n_keys[0] + B - 1; kv_per_batch: each query's own) are not in the cache
//    yet: a workgroup whose key slice holds some of query b's new keys rounds
//    those tokens' K (RoPE'd) and V to q8 itself, keeps them in LDS and reads
//    them there instead of the cache; query b's workgroup stores its own
//    token's K and V at their slot (one writer per key).
// 3. 64-key tiles: scores (NT/64 lanes per key), online softmax per head,
//    p*v with the tile's V staged in LDS.
// 4. The unnormalised partial (sum p*v, m, l) per head goes to `part`; the
//    last workgroup of a (b, KV head) to finish (an atomic counter, reset by
//    that workgroup for the next launch) merges the splits:
//    O = sum_s e^(m_s - M) O_s / sum_s e^(m_s - M) l_s (attn_merge.comp:18-47).
// ---------------------------------------------------------------------------
struct AttnArgs {
    const float *q;  // query rows [B][q_stride]; with rope: raw q, k, v rows of each token
    int64_t q_stride;
    const float *bias, *q_norm, *k_norm;
    float eps;
    const float2 *rope_cs;
    int n_rot, neox, rope, append;
    KvLayer kv;
    int kv_per_batch, n_ctx, H, HKV;
    const int32_t *n_keys;
    float scale;
    float *part;    // [B][n_split][HKV] groups of G records [HD + 2], attn_group_floats(G, HD) floats apart
    int *counters;  // [B * HKV] at CTR_STRIDE ints apart, zero between launches
    float *out;     // [B][H * HD]
    uint8_t *act_out;    // or null: the output also as matmul activation records (multi-query kernel)
    int64_t act_stride;  // bytes between tokens' records
    int win;             // > 0: a query sees only its last win keys (a sliding layer)
};

constexpr int ATTN_MAX_SPLIT = 64;
constexpr int ATTN_TILE = 64;

// Where work item (split, kvh, b) of n_split reads keys: [p0, p1) of the
// keys [lo, nk) of query b (at position pq = nk - 1; lo = 0, or nk - win for a
// sliding window of win keys), in 64-key tiles.
struct AttnSpan {
    int pq, p0, p1;
    int used;           // splits that hold keys: the others (later ones) are empty
    int64_t head_base;  // cache slot of key 0 for this KV head
    int n_lo, n_hi;     // the new keys (append) in this slice: [n_lo, n_hi)
    bool has_new;       // n_lo < n_hi
};
template <int TILE = ATTN_TILE>
__device__ inline AttnSpan attn_span(const AttnArgs &a, int split, int kvh, int b, int n_split) {
    AttnSpan sp;
    const int nk = a.kv_per_batch ? a.n_keys[b] : a.n_keys[0] + b + 1;
    sp.pq = nk - 1;
    const int lo = a.win > 0 ? max(0, nk - a.win) : 0, nw = nk - lo;
    // At least ATTN_MIN_KEYS keys a split: a short cache (or a small model's
    // few KV heads) leaves the later splits empty rather than merging many
    // slivers; an empty split's work item returns at once, and the merge
    // counts and reads the `used` ones only.
    int chunk = nw <= ATTN_SINGLE_MAX ? nw : max((nw + n_split - 1) / n_split, ATTN_MIN_KEYS);
    chunk = (chunk + TILE - 1) / TILE * TILE;
    sp.used = (nw + chunk - 1) / chunk;
    sp.p0 = lo + split * chunk;
    sp.p1 = min(nk, sp.p0 + chunk);
    const int seq = a.kv_per_batch ? b : 0;
    sp.head_base = ((int64_t)seq * a.HKV + kvh) * a.n_ctx;
    const int first = a.kv_per_batch ? sp.pq : a.n_keys[0];  // the batch's first new key
    // A slice that ends before the first new key holds none: n_hi = n_lo, not
    // below it (the preparation counts n_hi - n_lo new keys beside the query
    // heads it normalizes).
    sp.n_lo = max(first, sp.p0), sp.n_hi = a.append ? max(sp.n_lo, min(sp.pq + 1, sp.p1)) : sp.n_lo;
    sp.has_new = sp.n_lo < sp.n_hi;
    return sp;
}

// Inputs of the preparation of one query with at most one new key, loaded
// ahead (attn_preload) so that they return before loads issued after them:
// thread t's query values t, t + NT, ..., its values of the new key's K and V,
// and the RoPE table entries of its query and key pairs.
template <int HD, int G, int NT>
struct AttnPre {
    static constexpr int QK = (G * HD + NT - 1) / NT, KK = (2 * HD + NT - 1) / NT;
    static constexpr int QP = (G * (HD / 2) + NT - 1) / NT, KP = (HD / 2 + NT - 1) / NT;
    float q[QK], kv[KK];
    float2 qcs[QP], kcs[KP];
};
template <int HD, int G, int NT>
__device__ inline void attn_preload(const AttnArgs &a, int kvh, int b, const AttnSpan &sp, AttnPre<HD, G, NT> &p) {
    using P = AttnPre<HD, G, NT>;
    const int tid = threadIdx.x, pq = sp.pq, nn = sp.n_hi - sp.n_lo, nr2 = a.n_rot / 2;
    const float *qrow = a.q + (int64_t)b * a.q_stride;
#pragma unroll
    for (int k = 0; k < P::QK; k++) {
        const int j = tid + NT * k;
        const int64_t e = (int64_t)(kvh * G + min(j, G * HD - 1) / HD) * HD + j % HD;
        p.q[k] = j < G * HD ? qrow[e] + (a.rope && a.bias ? a.bias[e] : 0.f) : 0.f;
    }
#pragma unroll
    for (int k = 0; k < P::KK; k++) {
        const int j = tid + NT * k, which = (j / HD) & 1, d = j % HD;
        const int64_t e = (int64_t)((which ? a.H + a.HKV : a.H) + kvh) * HD + d;
        p.kv[k] = j < nn * 2 * HD ? qrow[e] + (a.bias ? a.bias[e] : 0.f) : 0.f;  // the new key is query b's own
    }
    if (a.rope) {
#pragma unroll
        for (int k = 0; k < P::QP; k++) {
            const int i = (tid + NT * k) % (HD / 2);
            p.qcs[k] = tid + NT * k < G * (HD / 2) && i < nr2 ? a.rope_cs[(int64_t)pq * nr2 + i] : make_float2(1.f, 0.f);
        }
#pragma unroll
        for (int k = 0; k < P::KP; k++) {
            const int i = tid + NT * k;
            p.kcs[k] = i < nn * nr2 ? a.rope_cs[(int64_t)sp.n_lo * nr2 + i] : make_float2(1.f, 0.f);
        }
    }
}

// 1. The G query heads of KV head kvh into LDS from query b's row; bias,
//    per-head norm and RoPE when a.rope. Then each new key of the slice
//    (n_lo .. n_hi - 1; the rows of those tokens, query b's row for key pq),
//    rounded as the cache keeps it (q8, or f16 with F16) into LDS slot
//    j - n_lo, and query b's own (pq) stored at its cache slot.
//    With `pre`: the query's inputs from there, and the new key's when the
//    slice's only new key is the query's own.
template <int HD, int G, int NT, bool F16, class Lds>
__device__ inline void attn_prepare(const AttnArgs &a, int kvh, int b, const AttnSpan &sp, Lds &S,
                                    const AttnPre<HD, G, NT> *pre = nullptr) {
    using P = AttnPre<HD, G, NT>;
    constexpr int NWV = NT / 64;
    auto &q_s = S.q_s;
    auto &kv_s = S.kv_s;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pq = sp.pq;
    const int nn = sp.n_hi - sp.n_lo;  // new keys in the slice, prepared together with the query
    const bool pre_kv = pre && (nn == 0 || (nn == 1 && sp.n_lo == pq));
    const float *qrow = a.q + (int64_t)b * a.q_stride;
    if (pre) {
#pragma unroll
        for (int k = 0; k < P::QK; k++) {
            const int j = tid + NT * k;
            if (j < G * HD) q_s[j / HD][j % HD] = pre->q[k];
        }
    } else {
        for (int j = tid; j < G * HD; j += NT) {
            const int64_t e = (int64_t)(kvh * G + j / HD) * HD + j % HD;
            q_s[j / HD][j % HD] = qrow[e] + (a.rope && a.bias ? a.bias[e] : 0.f);
        }
    }
    if (pre_kv) {
#pragma unroll
        for (int k = 0; k < P::KK; k++) {
            const int j = tid + NT * k;
            if (j < nn * 2 * HD) kv_s[0][(j / HD) & 1][j % HD] = pre->kv[k];
        }
    } else {
        for (int j = tid; j < nn * 2 * HD; j += NT) {
            const int kk = j / (2 * HD), which = (j / HD) & 1, d = j % HD;
            const float *row = a.q + (int64_t)(b - (pq - (sp.n_lo + kk))) * a.q_stride;  // the token at that position
            const int64_t e = (int64_t)((which ? a.H + a.HKV : a.H) + kvh) * HD + d;
            kv_s[kk][which][d] = row[e] + (a.bias ? a.bias[e] : 0.f);
        }
    }
    if (tid < G) {
        S.m_s[tid] = -INFINITY;
        S.l_s[tid] = 0.f;
    }
    __syncthreads();
    if (a.rope) {
        // Per-head RMSNorm (qwen3's q_norm, k_norm), then RoPE: the query
        // heads at the query's position, each key at its own.
        if (a.q_norm || (nn && a.k_norm)) {
            for (int g = wave; g < G + nn; g += NWV) {
                const float *nw = g < G ? a.q_norm : a.k_norm;
                if (!nw) continue;
                float *v = g < G ? q_s[g] : kv_s[g - G][0];
                float ss = 0.f;
                for (int j = lane; j < HD; j += 64) ss += v[j] * v[j];
                ss = wave_sum(ss);
                const float sc = 1.0f / sqrtf(ss / (float)HD + a.eps);
                for (int j = lane; j < HD; j += 64) v[j] = v[j] * sc * nw[j];
            }
            __syncthreads();
        }
        const int nr2 = a.n_rot / 2;
        auto rot = [&](float *v, int i, float2 cs) {
            const int i0 = a.neox ? i : 2 * i, i1 = a.neox ? i + nr2 : 2 * i + 1;
            float x0 = v[i0], x1 = v[i1];
            rope_pair(x0, x1, cs.x, cs.y);
            v[i0] = x0, v[i1] = x1;
        };
        if (pre) {
#pragma unroll
            for (int k = 0; k < P::QP; k++) {
                const int j = tid + NT * k, i = j % (HD / 2);
                if (j < G * (HD / 2) && i < nr2) rot(q_s[j / (HD / 2)], i, pre->qcs[k]);
            }
        } else {
            for (int j = tid; j < G * (HD / 2); j += NT) {
                const int g = j / (HD / 2), i = j % (HD / 2);
                if (i < nr2) rot(q_s[g], i, a.rope_cs[(int64_t)pq * nr2 + i]);
            }
        }
        __syncthreads();
        if (pre_kv) {
#pragma unroll
            for (int k = 0; k < P::KP; k++) {
                const int i = tid + NT * k;
                if (i < nn * nr2) rot(kv_s[0][0], i, pre->kcs[k]);
            }
        } else {
            for (int j = tid; j < nn * nr2; j += NT) {
                const int kk = j / nr2, i = j % nr2;
                rot(kv_s[kk][0], i, a.rope_cs[(int64_t)(sp.n_lo + kk) * nr2 + i]);
            }
        }
        __syncthreads();
    }
    if (nn == 0) return;
    // Rounded as the cache keeps them, a wave per (key, K or V), a pair of
    // values a lane; query b's own token (pq) also stored at its slot.
    for (int pr = wave; pr < 2 * nn; pr += NWV) {
        const int kk = pr >> 1, which = pr & 1, key = sp.n_lo + kk;
        const bool own = key == pq;
        const int64_t slot = sp.head_base + key;
        // Values d, d + 1 a lane: d = 2 lane (+ 128 past head dimension 128).
        for (int d = 2 * lane; d < HD; d += 128) {
        const int i = d / 2;
        if constexpr (F16) {  // engine/src/cpu_backend.cpp:80: each value to the nearest f16
            const uint32_t pair = (uint32_t)f2h(kv_s[kk][which][2 * i]) | (uint32_t)f2h(kv_s[kk][which][2 * i + 1]) << 16;
            *(uint32_t *)(S.new16[kk][which] + 2 * i) = pair;
            if (own) *(uint32_t *)((uint16_t *)(which ? a.kv.v : a.kv.k) + slot * HD + 2 * i) = pair;
        } else {
            // q8 (engine/src/cpu_backend.cpp:78-90): per 32 values sc = f16(amax / 127),
            // q = clamp(rint(v / sc), +-127).
            const float a0 = kv_s[kk][which][2 * i], a1 = kv_s[kk][which][2 * i + 1];
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
            const uint16_t packed = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
            *(uint16_t *)(S.new8[kk][which] + 2 * i) = packed;
            if (own) *(uint16_t *)((which ? a.kv.v : a.kv.k) + slot * HD + 2 * i) = packed;
            if ((i & 15) == 0) {
                S.new_sc[kk][which][i / 16] = sh;
                if (own) (which ? a.kv.vs : a.kv.ks)[slot * (HD / 32) + i / 16] = sh;
            }
        }
        }
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// One work item (split, KV head kvh, query b) of n_split over its key slice
// [p0, p1). Each wave walks its own keys with its own online softmax, with
// no workgroup barrier until the end:
//   lanes    LPK lanes a key, DPL dims a lane (16 with HD 128 and G <= 4,
//            else 8); KPS = 64 / LPK keys side by side a sweep, S sweeps a
//            chunk of 16 keys; the G query heads' DPL dims stay in registers;
//   chunks   a wave's chunk is 32 consecutive keys of the workgroup's chunk
//            of 32 * (NT / 64); the next chunk's K and V are requested before
//            the current one is used (buffer loads bounded by the slice: past
//            p1 they return zeros and touch no memory);
//   scores   DPL-dim partial dots added over the key's LPK lanes by DPP;
//   softmax  per head, the chunk's maximum over the wave, then
//            p = e^(s - m) and the running (m, l);
//   p * v    each lane adds p * v over its keys for its DPL dims; the keys of
//            other lanes are added once at the end.
// The waves' (m, l, o) then combine in LDS into the work item's partial, and
// the last of the n_split work items of a (query, KV head) to finish merges
// the partials (attn_merge.comp:18-47), reading them device-coherent.
// ---------------------------------------------------------------------------
template <int HD, int G>
struct SliceShape {
    static constexpr int DPL = (HD == 256 || (HD == 128 && G <= 4)) ? 16 : 8;  // dims a lane
    static constexpr int LPK = HD / DPL;                         // lanes a key: 8 or 16
    static constexpr int KPS = 64 / LPK;                         // keys a sweep: 8 or 4
    static constexpr int S = 16 / KPS;                           // sweeps a chunk (16 keys)
    static_assert(LPK == 8 || LPK == 16, "attention lane shape");
};

template <int HD, int G, int NT = 256>
struct SliceLds {
    float q_s[G][HD];
    float m_s[G], l_s[G], red[G];
    // The new keys' K and V before rounding live until the preparation's
    // last barrier; the waves' results are written after it: one space.
    union {
        float kv_s[ATTN_MAX_NEW][2][HD];
        struct {
            __align__(16) float o_w[NT / 64][G][HD];  // each wave's o
            float m_w[NT / 64][G], l_w[NT / 64][G];   // ... and (m, l)
        };
    };
    // The rounded new keys: int8 with f16 scales (a q8 cache) or f16.
    union {
        struct {
            __align__(16) int8_t new8[ATTN_MAX_NEW][2][HD];
            uint16_t new_sc[ATTN_MAX_NEW][2][HD / 32];
        };
        __align__(16) uint16_t new16[ATTN_MAX_NEW][2][HD];
    };
    __align__(16) float wts[G][ATTN_MAX_SPLIT];  // the merge's weight per (head, split), 0 past n_split
    int last;
};

// The cache's values: q8 (int8 with an f16 scale per 32) or, with F16, f16
// (2 bytes a value, no scales; ks / vs unused).
template <bool F16>
__device__ inline float kv_value(const uint32_t *w, int e) {
    if constexpr (F16) return h2f((w[e >> 1] >> (16 * (e & 1))) & 0xffff);
    else return (float)(int8_t)((w[e >> 2] >> (8 * (e & 3))) & 0xff);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// A buffer resource over [base, base + bytes): loads past the end return 0
// without a memory access (gfx9 raw buffers).
__device__ inline __amdgpu_buffer_rsrc_t slice_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}
template <int BYTES>
struct Raw {
    uint32_t w[BYTES / 4];
};
template <int BYTES>
__device__ inline Raw<BYTES> buf_load(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    Raw<BYTES> v;
    if constexpr (BYTES == 32) {
        const auto a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
        const auto b = __builtin_amdgcn_raw_buffer_load_b128(r, off + 16, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) v.w[i] = a[i], v.w[4 + i] = b[i];
    } else if constexpr (BYTES == 16) {
        const auto a = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) v.w[i] = a[i];
    } else {
        static_assert(BYTES == 8, "buffer load size");
        const auto a = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
        v.w[0] = a[0], v.w[1] = a[1];
    }
    return v;
}

// ---------------------------------------------------------------------------
// Split partials and their merge, shared by k_attn and k_attn_lds. Per
// (query b, split, KV head) a group of attn_group_floats(G, HD) floats (whole
// 128-byte lines): the G heads' unnormalised output sums [G][HD], then (m, l)
// per head. A KV head's splits run on every XCD (workgroups go to the XCDs
// in turn), so partials are written and read device-coherent: buffer
// accesses with sc1 (stores through to memory, loads past this XCD's L2).
// They are 16 bytes a lane: the merging work item then reads the 32 splits
// of a 4-head group (66 KB) in about half the time 4-byte loads take (0.8
// against 1.6 us); it is the one work item left on the KV head's critical
// path, so its read is issue-bound, not bandwidth-bound.
// ---------------------------------------------------------------------------
constexpr int BUF_SC1 = 16;  // buffer cache policy: sc1 (device coherent)

template <int G, int HD>
__device__ inline float *attn_part_group(const AttnArgs &a, int b, int split, int kvh, int n_split) {
    return a.part + (((int64_t)b * n_split + split) * a.HKV + kvh) * (int64_t)attn_group_floats(G, HD);
}

// Writes this work item's partial: quad q of the sums is sums(q) (values 4q ..
// 4q + 3), head g's (m, l) is ml(g). Returns when the stores are complete.
template <int G, int HD, int NT, class Sums, class ML>
__device__ inline void attn_publish(float *pb, Sums sums, ML ml) {
    constexpr int NOUT = G * HD;
    const __amdgpu_buffer_rsrc_t r = slice_rsrc(pb, (uint32_t)attn_group_floats(G, HD) * 4);
    for (int q = threadIdx.x; q < NOUT / 4; q += NT)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sums(q)), r, (uint32_t)q * 16, 0, BUF_SC1);
    if (threadIdx.x < G) {
        const float2 v = ml((int)threadIdx.x);
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), r, (uint32_t)(NOUT + 2 * threadIdx.x) * 4,
                                              0, BUF_SC1);
    }
    wait_stores();
}

// The merge, by the work item that counted a KV head's `used` splits last:
// every split's (m, l) becomes a weight (a wave a head, a lane a split: wts,
// red), then threads in SETS sets each add up quads of the output over their
// share of the splits, all of a batch's loads requested together; the sets'
// sums meet in LDS (xs: (SETS - 1) * G * HD floats, free by now) and the
// first set writes the G heads' outputs. Leaves the KV head's counter zero.
template <int G, int HD, int NT>
__device__ inline void attn_merge(const AttnArgs &a, int b, int kvh, int n_split, int used,
                                  float (&wts)[G][ATTN_MAX_SPLIT], float *red, float *xs) {
    constexpr float LOG2E = 1.4426950408889634f;
    constexpr int NOUT = G * HD, NQ4 = NOUT / 4, NW = NT / 64;
    constexpr int SETS = NT / NQ4 < 1 ? 1 : (NT / NQ4 > NW ? NW : NT / NQ4);
    constexpr int PER = (NQ4 + NT - 1) / NT;  // quads a thread (SETS 1 with more quads than threads)
    constexpr int MB = 32 / SETS;             // loads a thread per quad and batch: 32 splits a batch in all
    constexpr int64_t grp = attn_group_floats(G, HD);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int set = SETS > 1 ? tid / NQ4 : 0, tq = SETS > 1 ? tid % NQ4 : tid;
    // Threads past the sets' quads only help with the weights.
    const bool active = SETS > 1 ? set < SETS : (PER > 1 || tid < NQ4);
    const float *p_all = a.part + ((int64_t)b * n_split * a.HKV + kvh) * grp;
    const int64_t sstride = (int64_t)a.HKV * grp;  // floats between splits
    const __amdgpu_buffer_rsrc_t rp = slice_rsrc(p_all, (uint32_t)((used - 1) * sstride + grp) * 4);
    u32x4 v[PER][MB];
    auto fetch = [&](int s0) {
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int q = min(tq + NT * k, NQ4 - 1);
#pragma unroll
            for (int i = 0; i < MB; i++) {
                const int sl = min(s0 + set + SETS * i, used - 1);
                v[k][i] = __builtin_amdgcn_raw_buffer_load_b128(rp, (uint32_t)((sl * sstride + 4 * q) * 4), 0, BUF_SC1);
            }
        }
    };
    if (active) fetch(0);
    for (int g = wave; g < G; g += NW) {
        const int sl = min(lane, used - 1);
        const u32x2 ml = __builtin_amdgcn_raw_buffer_load_b64(rp, (uint32_t)((sl * sstride + NOUT + 2 * g) * 4), 0, BUF_SC1);
        const float m0 = __uint_as_float(ml[0]), l0 = __uint_as_float(ml[1]);
        const float mm = lane < used ? m0 : -INFINITY;
        const float M = wave_max_dpp(mm);
        const float w = mm == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((mm - M) * LOG2E);
        const float L = wave_sum_dpp(w * (lane < used ? l0 : 0.f));
        wts[g][lane] = w;  // lanes past the used splits: 0
        if (lane == 0) red[g] = L;
    }
    __syncthreads();
    float4 acc[PER];
#pragma unroll
    for (int k = 0; k < PER; k++) acc[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (active) {
        for (int s0 = 0; s0 < used; s0 += 32) {
            if (s0) fetch(s0);
#pragma unroll
            for (int k = 0; k < PER; k++) {
                const int g = 4 * min(tq + NT * k, NQ4 - 1) / HD;
#pragma unroll
                for (int i = 0; i < MB; i++) {
                    const int sl = s0 + set + SETS * i;
                    const float w = sl < used ? wts[g][sl] : 0.f;
                    acc[k].x += w * __uint_as_float(v[k][i][0]);
                    acc[k].y += w * __uint_as_float(v[k][i][1]);
                    acc[k].z += w * __uint_as_float(v[k][i][2]);
                    acc[k].w += w * __uint_as_float(v[k][i][3]);
                }
            }
        }
    }
    if constexpr (SETS > 1) {
        if (active && set > 0) *(float4 *)&xs[(set - 1) * NOUT + 4 * tq] = acc[0];
        __syncthreads();
        if (set == 0)
#pragma unroll
            for (int s2 = 1; s2 < SETS; s2++) {
                const float4 o = *(const float4 *)&xs[(s2 - 1) * NOUT + 4 * tq];
                acc[0].x += o.x, acc[0].y += o.y, acc[0].z += o.z, acc[0].w += o.w;
            }
    }
    if (set == 0) {
#pragma unroll
        for (int k = 0; k < PER; k++) {
            const int q = tq + NT * k;
            if (q < NQ4) {
                const float L = red[4 * q / HD];
                const float4 r = L > 0.f ? make_float4(acc[k].x / L, acc[k].y / L, acc[k].z / L, acc[k].w / L)
                                         : make_float4(0.f, 0.f, 0.f, 0.f);
                *(float4 *)(a.out + (int64_t)b * a.H * HD + (int64_t)kvh * G * HD + 4 * q) = r;
            }
        }
    }
    if (tid == 0) st_dev(a.counters + (b * a.HKV + kvh) * CTR_STRIDE, 0);  // ready for the next use
}

// The end of a work item: its (m, l, o) from its waves' (S.m_w, S.l_w,
// S.o_w: [wave][head] with m in the natural-log domain), then the output
// itself when it is the only split with keys, else its partial, the count,
// and the merge by the last work item of the (query, KV head).
template <int HD, int G, int NT, class Lds>
__device__ inline void attn_item_out(const AttnArgs &a, const AttnSpan &sp, int split, int kvh, int b, int n_split,
                                     Lds &S) {
    constexpr int NW = NT / 64;
    constexpr float LOG2E = 1.4426950408889634f;
    const int tid = threadIdx.x;
    constexpr int NOUT = G * HD;
    auto item_value = [&](int j, float &mo, float &lo_) -> float {
        const int g = j / HD, d = j % HD;
        float M = S.m_w[0][g];
#pragma unroll
        for (int w = 1; w < NW; w++) M = fmaxf(M, S.m_w[w][g]);
        float O = 0.f, L = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float wt = S.m_w[w][g] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((S.m_w[w][g] - M) * LOG2E);
            O += wt * S.o_w[w][g][d];
            L += wt * S.l_w[w][g];
        }
        mo = M, lo_ = L;
        return O;
    };
    if (sp.used == 1) {  // the only split with keys: the output directly, as the merge would
        for (int j = tid; j < NOUT; j += NT) {
            float M, L;
            const float O = item_value(j, M, L);
            a.out[(int64_t)b * a.H * HD + (int64_t)kvh * G * HD + j] = L > 0.f ? O / L : 0.f;
        }
        return;
    }
    attn_publish<G, HD, NT>(
        attn_part_group<G, HD>(a, b, split, kvh, n_split),
        [&](int q) {
            float M, L, o[4];
#pragma unroll
            for (int i = 0; i < 4; i++) o[i] = item_value(4 * q + i, M, L);
            return make_float4(o[0], o[1], o[2], o[3]);
        },
        [&](int g) {
            float M, L;
            item_value(g * HD, M, L);
            return make_float2(M, L);
        });
    __syncthreads();
    if (tid == 0) S.last = atomicAdd(a.counters + (b * a.HKV + kvh) * CTR_STRIDE, 1) == sp.used - 1;
    __syncthreads();
    if (!S.last) return;
    attn_merge<G, HD, NT>(a, b, kvh, n_split, sp.used, S.wts, S.red, &S.o_w[0][0][0]);
}

template <int HD, int G, int NT, bool F16 = false>
__device__ inline void attn_slice(const AttnArgs &a, int split, int kvh, int b, int n_split,
                                  SliceLds<HD, G, NT> &S) {
    using SH = SliceShape<HD, G>;
    constexpr int NW = NT / 64, DPL = SH::DPL, LPK = SH::LPK, KPS = SH::KPS, NS = SH::S;
    constexpr int VB = F16 ? 2 : 1;         // bytes per cached value
    constexpr int RB = DPL * VB;            // bytes of a key a lane reads
    constexpr int WCH = NS * KPS, GCH = NW * WCH;  // keys a wave chunk, a workgroup chunk
    constexpr float LOG2E = 1.4426950408889634f;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ks_ = lane / LPK, dq = lane % LPK;  // key slot of a sweep, dim quarter
    const int d0 = DPL * dq;
    const AttnSpan sp = attn_span<16>(a, split, kvh, b, n_split);
    if (split >= sp.used) return;  // an empty split: not counted, not merged
    const int nkeys = max(sp.p1 - sp.p0, 0);
    // The slice's K and V (and scales) as bounded buffers from key p0.
    const int8_t *kb = a.kv.k + (sp.head_base + sp.p0) * HD * VB, *vb = a.kv.v + (sp.head_base + sp.p0) * HD * VB;
    const __amdgpu_buffer_rsrc_t rk = slice_rsrc(kb, (uint32_t)nkeys * HD * VB);
    const __amdgpu_buffer_rsrc_t rv = slice_rsrc(vb, (uint32_t)nkeys * HD * VB);
    __amdgpu_buffer_rsrc_t rks = rk, rvs = rv;
    if constexpr (!F16) {
        rks = slice_rsrc(a.kv.ks + (sp.head_base + sp.p0) * (HD / 32), (uint32_t)nkeys * (HD / 32) * 2);
        rvs = slice_rsrc(a.kv.vs + (sp.head_base + sp.p0) * (HD / 32), (uint32_t)nkeys * (HD / 32) * 2);
    }
    struct Chunk {
        Raw<RB> k[NS], v[NS];
        uint32_t ks[NS], vs[NS];
    };
    // Chunk c of the slice, this wave's 16 keys: key (relative to p0)
    // c * GCH + wave * WCH + s * KPS + ks_.
    auto request = [&](Chunk &ch, int c) {
#pragma unroll
        for (int s2 = 0; s2 < NS; s2++) {
            const uint32_t key = (uint32_t)(c * GCH + wave * WCH + s2 * KPS + ks_);
            const uint32_t off = (key * HD + d0) * VB;
            ch.k[s2] = buf_load<RB>(rk, off);
            ch.v[s2] = buf_load<RB>(rv, off);
            if constexpr (!F16) {
                const uint32_t so = (key * (HD / 32) + d0 / 32) * 2;
                ch.ks[s2] = __builtin_amdgcn_raw_buffer_load_b16(rks, so, 0, 0);
                ch.vs[s2] = __builtin_amdgcn_raw_buffer_load_b16(rvs, so, 0, 0);
            }
        }
    };
    Chunk buf[ATTN_DEPTH];
#pragma unroll
    for (int i = 0; i < ATTN_DEPTH; i++) request(buf[i], i);
    attn_prepare<HD, G, NT, F16>(a, kvh, b, sp, S);
    float q[G][DPL], o[G][DPL], m[G], l[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
#pragma unroll
        for (int e = 0; e < DPL; e += 4) {
            const float4 v = *(const float4 *)&S.q_s[g][d0 + e];
            q[g][e] = v.x, q[g][e + 1] = v.y, q[g][e + 2] = v.z, q[g][e + 3] = v.w;
        }
#pragma unroll
        for (int e = 0; e < DPL; e++) o[g][e] = 0.f;
        m[g] = -INFINITY, l[g] = 0.f;
    }
    const int nlo_rel = sp.n_lo - sp.p0, nnew = sp.n_hi - sp.n_lo;  // the new keys, relative to p0
    // One chunk: scores, softmax update, p * v.
    auto consume = [&](Chunk &ch, int c) {
        // Whether a new key is among this wave's 16 (the same for the whole
        // wave).
        const int cb = c * GCH + wave * WCH;
        const bool new_here = sp.has_new && cb < nlo_rel + nnew && nlo_rel < cb + WCH;
        float sc[NS][G];
#pragma unroll
        for (int s2 = 0; s2 < NS; s2++) {
            const int key = c * GCH + wave * WCH + s2 * KPS + ks_;
            uint32_t kw[RB / 4];
#pragma unroll
            for (int i = 0; i < RB / 4; i++) kw[i] = ch.k[s2].w[i];
            float kscale = F16 ? 1.f : h2f(ch.ks[s2]);
            if (new_here && (unsigned)(key - nlo_rel) < (unsigned)nnew) {  // a new key, from LDS
                const int jj = key - nlo_rel;
#pragma unroll
                for (int i = 0; i < RB / 4; i++)
                    kw[i] = F16 ? *(const uint32_t *)(S.new16[jj][0] + d0 + 2 * i)
                                : *(const uint32_t *)(S.new8[jj][0] + d0 + 4 * i);
                if constexpr (!F16) kscale = h2f(S.new_sc[jj][0][d0 / 32]);
            }
            float acc[G];
#pragma unroll
            for (int g = 0; g < G; g++) acc[g] = 0.f;
#pragma unroll
            for (int e = 0; e < DPL; e++) {
                const float kf = kv_value<F16>(kw, e);
#pragma unroll
                for (int g = 0; g < G; g++) acc[g] += q[g][e] * kf;
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                // Each lane's dims lie in one 32-value block of the key: its
                // own scale before the key's lanes are added.
                float v = acc[g] * kscale;
                v = dpp_add<0xB1, 0xF, true>(v);   // quad_perm [1,0,3,2]
                v = dpp_add<0x4E, 0xF, true>(v);   // quad_perm [2,3,0,1]
                v = dpp_add<0x141, 0xF, true>(v);  // row_half_mirror: the 8 lanes
                if constexpr (LPK == 16) v = dpp_add<0x140, 0xF, true>(v);  // row_mirror: 16
                sc[s2][g] = key < nkeys ? v * a.scale : -INFINITY;
            }
        }
        // The chunk's largest score per head over the wave's key slots.
        float alpha[G], p[NS][G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float cm = sc[0][g];
#pragma unroll
            for (int s2 = 1; s2 < NS; s2++) cm = fmaxf(cm, sc[s2][g]);
            if constexpr (LPK == 8) cm = dpp_max<0x128, 0xF, true>(cm);  // row_ror:8
            {
                const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(cm), __float_as_uint(cm), false, false);
                cm = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
                const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(cm), __float_as_uint(cm), false, false);
                cm = fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
            }
            const float mn = fmaxf(m[g], cm);
            alpha[g] = m[g] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m[g] - mn) * LOG2E);
            float ls = 0.f;
#pragma unroll
            for (int s2 = 0; s2 < NS; s2++) {
                p[s2][g] = sc[s2][g] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((sc[s2][g] - mn) * LOG2E);
                ls += p[s2][g];
            }
            if constexpr (LPK == 8) ls = dpp_add<0x128, 0xF, true>(ls);
            ls = add_xor32(add_xor16(ls));
            m[g] = mn;
            l[g] = l[g] * alpha[g] + ls;
        }
        bool same = true;  // no head's maximum moved: o stays as it is
#pragma unroll
        for (int g = 0; g < G; g++) same = same && alpha[g] == 1.f;
        if (!same) {
#pragma unroll
            for (int g = 0; g < G; g++)
#pragma unroll
                for (int e = 0; e < DPL; e++) o[g][e] *= alpha[g];
        }
#pragma unroll
        for (int s2 = 0; s2 < NS; s2++) {
            const int key = c * GCH + wave * WCH + s2 * KPS + ks_;
            uint32_t vw[RB / 4];
#pragma unroll
            for (int i = 0; i < RB / 4; i++) vw[i] = ch.v[s2].w[i];
            float vscale = F16 ? 1.f : h2f(ch.vs[s2]);
            if (new_here && (unsigned)(key - nlo_rel) < (unsigned)nnew) {
                const int jj = key - nlo_rel;
#pragma unroll
                for (int i = 0; i < RB / 4; i++)
                    vw[i] = F16 ? *(const uint32_t *)(S.new16[jj][1] + d0 + 2 * i)
                                : *(const uint32_t *)(S.new8[jj][1] + d0 + 4 * i);
                if constexpr (!F16) vscale = h2f(S.new_sc[jj][1][d0 / 32]);
            }
            float w[G];
#pragma unroll
            for (int g = 0; g < G; g++) w[g] = p[s2][g] * vscale;
#pragma unroll
            for (int e = 0; e < DPL; e++) {
                const float vf = kv_value<F16>(vw, e);
#pragma unroll
                for (int g = 0; g < G; g++) o[g][e] += w[g] * vf;
            }
        }
    };
    // ATTN_DEPTH register buffers in turn, all requested before the query
    // is prepared; each is refilled with the chunk ATTN_DEPTH on as soon as
    // it is consumed (past the slice: no memory access).
    const int nch = (nkeys + GCH - 1) / GCH;
    for (int c = 0; c < nch; c += ATTN_DEPTH) {
#pragma unroll
        for (int i = 0; i < ATTN_DEPTH; i++) {
            if (c + i >= nch) break;
            consume(buf[i], c + i);
            request(buf[i], c + i + ATTN_DEPTH);
        }
    }
    // The key slots of a wave hold the same dims: add them over lanes i ^ 32,
    // i ^ 16 (and i ^ 8 within a 16-lane row when LPK is 8) by a butterfly
    // that pairs different values in each swap: v_permlane32_swap of (a, b)
    // leaves a's pair sums in lanes 0-31 and b's in lanes 32-63, and
    // v_permlane16_swap does the same for rows 0 / 1 and 2 / 3. The NV values
    // end as NV / 4 registers, row r of register i holding value
    // i + (NV / 4) r summed over every slot.
    constexpr int NV = G * DPL, N2 = NV / 2, N4 = NV / 4;
    static_assert(NV % 4 == 0, "o butterfly");
    float r2[N4];
    {
        float r1[N2];
#pragma unroll
        for (int i = 0; i < N2; i++) {
            const float x = o[i / DPL][i % DPL], y = o[(i + N2) / DPL][(i + N2) % DPL];
            const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
            r1[i] = __uint_as_float(t[0]) + __uint_as_float(t[1]);
        }
#pragma unroll
        for (int i = 0; i < N4; i++) {
            const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(r1[i]), __float_as_uint(r1[i + N4]), false, false);
            float v = __uint_as_float(t[0]) + __uint_as_float(t[1]);
            if constexpr (LPK == 8) v = dpp_add<0x128, 0xF, true>(v);  // row_ror:8
            r2[i] = v;
        }
    }
    if ((lane & 15) < LPK) {  // row r, dims of lane % LPK
        const int row = lane >> 4;
#pragma unroll
        for (int i = 0; i < N4; i++) {
            const int j = i + N4 * row, g = j / DPL, e = j % DPL;
            S.o_w[wave][g][d0 + e] = r2[i];
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) S.m_w[wave][g] = m[g], S.l_w[wave][g] = l[g];
    }
    __syncthreads();

    attn_item_out<HD, G, NT>(a, sp, split, kvh, b, n_split, S);
}

// The matrix-core one-query kernel (attn_m1.hip): G query heads a KV head,
// a q8 or f16 cache at head dimension 128, grid (n_split, HKV, B).
hipError_t launch_attn_m1(int G, bool f16, dim3 grid, const AttnArgs &a, hipStream_t s);

}  // namespace ts5hip
