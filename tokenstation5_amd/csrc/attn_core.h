// Device core of split-K flash decode over the KV cache (q8, or f16), used
// by the kernels of attention.hip.
#pragma once
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace ts5hip {

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
// 2. `append` (B == 1): the workgroup whose key slice holds the new key
//    rounds that token's K (RoPE'd) and V to q8, stores them at their slot,
//    and keeps a copy in LDS that it reads instead of the cache.
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
};

__device__ inline void rope_inplace(float *v, int n_rot, int neox, const float2 *cs, int i) {
    const int a = neox ? i : 2 * i, b = neox ? i + n_rot / 2 : 2 * i + 1;
    float x0 = v[a], x1 = v[b];
    rope_pair(x0, x1, cs[i].x, cs[i].y);
    v[a] = x0;
    v[b] = x1;
}

constexpr int ATTN_MAX_SPLIT = 64;
constexpr int ATTN_TILE = 64;

// K bytes per lane of a key's score: NQ = HD / (NT / 64) lanes' worth.
template <int NQ>
struct KRow {
    uint32_t w[NQ / 4];
};
template <int NQ>
__device__ inline KRow<NQ> load_krow(const int8_t *p) {
    KRow<NQ> r;
    if constexpr (NQ % 16 == 0) {
#pragma unroll
        for (int c = 0; c < NQ / 16; c++) {
            const uint4 v = *(const uint4 *)(p + 16 * c);
            r.w[4 * c] = v.x, r.w[4 * c + 1] = v.y, r.w[4 * c + 2] = v.z, r.w[4 * c + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int c = 0; c < NQ / 8; c++) {
            const uint2 v = *(const uint2 *)(p + 8 * c);
            r.w[2 * c] = v.x, r.w[2 * c + 1] = v.y;
        }
    }
    return r;
}

// Where work item (split, kvh, b) of n_split reads keys: [p0, p1) of the nk
// keys [0, nk) of query b (at position pq = nk - 1), in 64-key tiles.
struct AttnSpan {
    int pq, p0, p1;
    int64_t head_base;  // cache slot of key 0 for this KV head
    bool has_new;       // the new key (pq) falls in this slice
};
template <int TILE = ATTN_TILE>
__device__ inline AttnSpan attn_span(const AttnArgs &a, int split, int kvh, int b, int n_split) {
    AttnSpan sp;
    const int nk = a.kv_per_batch ? a.n_keys[b] : a.n_keys[0] + b + 1;
    sp.pq = nk - 1;
    int chunk = (nk + n_split - 1) / n_split;
    chunk = (chunk + TILE - 1) / TILE * TILE;
    sp.p0 = split * chunk;
    sp.p1 = min(nk, sp.p0 + chunk);
    const int seq = a.kv_per_batch ? b : 0;
    sp.head_base = ((int64_t)seq * a.HKV + kvh) * a.n_ctx;
    sp.has_new = a.append && sp.pq >= sp.p0 && sp.pq < sp.p1;
    return sp;
}

// 1. The G query heads of KV head kvh (and, when the slice holds the new key,
//    that token's K and V) into LDS, from q(e) = element e of the token's
//    q|k|v row; bias, per-head norm and RoPE when a.rope; the new K and V
//    rounded as the cache keeps them (q8, or f16 with F16) and stored at
//    their cache slot.
template <int HD, int G, int NT, bool F16, class QLoad, class Lds>
__device__ inline void attn_prepare(const AttnArgs &a, int kvh, const AttnSpan &sp, Lds &S, QLoad qload) {
    constexpr int NWV = NT / 64;
    auto &q_s = S.q_s;
    auto &kv_s = S.kv_s;
    auto &new8 = S.new8;
    auto &new_sc = S.new_sc;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int pq = sp.pq;
    const bool has_new = sp.has_new;
    for (int j = tid; j < G * HD; j += NT) {
        const int64_t e = (int64_t)(kvh * G + j / HD) * HD + j % HD;
        q_s[j / HD][j % HD] = qload(e) + (a.rope && a.bias ? a.bias[e] : 0.f);
    }
    if (has_new) {
        for (int j = tid; j < 2 * HD; j += NT) {
            const int64_t e = (int64_t)((j < HD ? a.H : a.H + a.HKV) + kvh) * HD + j % HD;
            kv_s[j / HD][j % HD] = qload(e) + (a.bias ? a.bias[e] : 0.f);
        }
    }
    if (tid < G) {
        S.m_s[tid] = -INFINITY;
        S.l_s[tid] = 0.f;
    }
    __syncthreads();
    if (a.rope) {
        // Per-head RMSNorm (qwen3's q_norm / k_norm), then RoPE.
        if (a.q_norm || (has_new && a.k_norm)) {
            for (int g = wave; g < G + 1; g += NWV) {
                const float *nw = g < G ? a.q_norm : (has_new ? a.k_norm : nullptr);
                if (!nw) continue;
                float *v = g < G ? q_s[g] : kv_s[0];
                float ss = 0.f;
                for (int j = lane; j < HD; j += 64) ss += v[j] * v[j];
                ss = wave_sum(ss);
                const float sc = 1.0f / sqrtf(ss / (float)HD + a.eps);
                for (int j = lane; j < HD; j += 64) v[j] = v[j] * sc * nw[j];
            }
            __syncthreads();
        }
        const float2 *cs = a.rope_cs + (int64_t)pq * (a.n_rot / 2);
        for (int j = tid; j < (G + 1) * (HD / 2); j += NT) {
            const int g = j / (HD / 2), i = j % (HD / 2);
            if (i >= a.n_rot / 2) continue;
            if (g < G) rope_inplace(q_s[g], a.n_rot, a.neox, cs, i);
            else if (has_new) rope_inplace(kv_s[0], a.n_rot, a.neox, cs, i);
        }
        __syncthreads();
    }
    if (F16 && has_new && tid < 128) {
        // f16 (engine/src/cpu_backend.cpp:80): each value rounded to the
        // nearest f16. Wave 0 rounds K, wave 1 V, a pair per lane.
        const int which = tid >> 6, i = tid & 63;
        if (2 * i < HD) {
            const uint32_t pair = (uint32_t)f2h(kv_s[which][2 * i]) | (uint32_t)f2h(kv_s[which][2 * i + 1]) << 16;
            const int64_t slot = sp.head_base + pq;
            *(uint32_t *)(S.new16[which] + 2 * i) = pair;
            *(uint32_t *)((uint16_t *)(which ? a.kv.v : a.kv.k) + slot * HD + 2 * i) = pair;
        }
    }
    if (!F16 && has_new && tid < 128) {
        // q8 (engine/src/cpu_backend.cpp:78-90): per 32 values sc = f16(amax / 127),
        // q = clamp(rint(v / sc), +-127). Wave 0 rounds K, wave 1 V, a pair per lane.
        const int which = tid >> 6, i = tid & 63;
        if (2 * i < HD) {
            const float a0 = kv_s[which][2 * i], a1 = kv_s[which][2 * i + 1];
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
            const int64_t slot = sp.head_base + pq;
            *(uint16_t *)(new8[which] + 2 * i) = packed;
            *(uint16_t *)((which ? a.kv.v : a.kv.k) + slot * HD + 2 * i) = packed;
            if ((i & 15) == 0) {
                new_sc[which][i / 16] = sh;
                (which ? a.kv.vs : a.kv.ks)[slot * (HD / 32) + i / 16] = sh;
            }
        }
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// One work item (split, KV head kvh, query b) of n_split over its whole key
// slice, in passes of up to ATTN_KT keys: every K and V byte of a pass is
// requested before the query's preparation and held in registers, so the
// slice costs one memory round trip rather than one per 64-key tile.
//   scores   4 lanes per key (HD/4 dims each), 64 keys per sweep of the
//            workgroup, q from LDS, the 4 partial sums added by DPP;
//   softmax  a wave per head over the pass, online across passes;
//   p * v    8 dims per lane straight from the V rows in registers, G heads
//            per V value; the lanes and waves that took other keys of the
//            same dims are added at the end (shuffles, then LDS).
// Then the partial record and the merge of attn_item.
// ---------------------------------------------------------------------------
constexpr int ATTN_KT = 256;

template <int HD, int G, int NT = 256>
struct SliceLds {
    float q_s[G][HD];
    __align__(16) float p_s[ATTN_KT][G];  // scores, then probabilities
    float alpha_s[G], m_s[G], l_s[G], red[G];
    float kv_s[2][HD];                    // the new token's K and V before rounding
    __align__(16) int8_t new8[2][HD];     // ... and after, as int8
    uint16_t new_sc[2][HD / 32];          // ... with their f16 scales
    __align__(16) uint16_t new16[2][HD];  // ... or as f16 (an f16 cache)
    __align__(16) float o_s[NT / 64][G * HD];  // each wave's p * v sums
    __align__(16) float wts[G][ATTN_MAX_SPLIT];  // the merge's weight per (head, split), 0 past n_split
    int last;
};

template <int HD, int G, int NT>
struct SliceShape {
    // Scores: LPK lanes a key, KS keys a sweep of the workgroup, NPASS sweeps a
    // pass. p * v: DPL dims a lane, KPW keys a wave, KPS keys a step, NVS steps.
    static constexpr int NW = NT / 64, LPK = 4, NQ = HD / LPK, KS = NT / LPK, NPASS = ATTN_KT / KS;
    static constexpr int DPL = 8, LPV = HD / DPL, KPW = 64 / LPV, KPS = NW * KPW, NVS = ATTN_KT / KPS;
    static_assert(NQ % 8 == 0 && LPV <= 64 && 64 % LPV == 0 && 64 % KPS == 0 && ATTN_KT % KS == 0,
                  "attention slice shape");
};

// The cache's values: q8 (int8 with an f16 scale per 32) or, with F16, f16
// (2 bytes a value, no scales; ks / vs unused). A lane's 8 V dims are one
// uint2 of int8 or one uint4 of f16.
template <bool F16>
using VRow = typename std::conditional<F16, uint4, uint2>::type;
template <bool F16>
__device__ inline float kv_value(const uint32_t *w, int e) {
    if constexpr (F16) return h2f((w[e >> 1] >> (16 * (e & 1))) & 0xffff);
    else return (float)(int8_t)((w[e >> 2] >> (8 * (e & 3))) & 0xff);
}

template <int HD, int G, int NT, bool F16 = false>
__device__ inline void attn_slice(const AttnArgs &a, int split, int kvh, int b, int n_split,
                                  SliceLds<HD, G, NT> &S) {
    using SH = SliceShape<HD, G, NT>;
    constexpr int NW = SH::NW, NQ = SH::NQ, KS = SH::KS, NPASS = SH::NPASS, LPV = SH::LPV, KPW = SH::KPW,
                  KPS = SH::KPS, NVS = SH::NVS, SMX = ATTN_KT / 64;
    constexpr int VB = F16 ? 2 : 1;  // bytes per cached value
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kk = tid >> 2, qq = tid & 3;              // scores: key kk of a sweep, quarter qq of the dims
    const int vk = lane / LPV, vc = lane % LPV;         // p * v: key vk of a wave's step, dims 8 vc ..
    const AttnSpan sp = attn_span<16>(a, split, kvh, b, n_split);
    const int8_t *kb = a.kv.k + sp.head_base * HD * VB, *vb = a.kv.v + sp.head_base * HD * VB;
    const uint16_t *ksb = F16 ? nullptr : a.kv.ks + sp.head_base * (HD / 32);
    const uint16_t *vsb = F16 ? nullptr : a.kv.vs + sp.head_base * (HD / 32);
    float o[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) o[g][e] = 0.f;
    bool prepared = false;
    for (int t0 = sp.p0; t0 < sp.p1 || !prepared; t0 += ATTN_KT) {
        const int nt = max(0, min(ATTN_KT, sp.p1 - t0));
        const int kmax = max(sp.p1 - 1, 0);  // loads past the slice read its last key (zero weight)
        KRow<NQ * VB> kr[NPASS];
        uint16_t ksr[NPASS];
#pragma unroll
        for (int j = 0; j < NPASS; j++) {
            const int key = min(t0 + KS * j + kk, kmax);
            kr[j] = load_krow<NQ * VB>(kb + ((int64_t)key * HD + qq * NQ) * VB);
            if constexpr (!F16) ksr[j] = ksb[(int64_t)key * (HD / 32) + (qq * NQ) / 32];
        }
        VRow<F16> vr[NVS];
        uint16_t vsr[NVS];
#pragma unroll
        for (int s2 = 0; s2 < NVS; s2++) {
            const int key = min(t0 + s2 * KPS + wave * KPW + vk, kmax);
            vr[s2] = *(const VRow<F16> *)(vb + ((int64_t)key * HD + 8 * vc) * VB);
            if constexpr (!F16) vsr[s2] = vsb[(int64_t)key * (HD / 32) + (8 * vc) / 32];
        }
        if (!prepared) {
            const float *row = a.q + (int64_t)b * a.q_stride;
            attn_prepare<HD, G, NT, F16>(a, kvh, sp, S, [&](int64_t e) { return row[e]; });
            prepared = true;
            if (nt == 0) break;
        }
        // Scores of the pass.
#pragma unroll
        for (int j = 0; j < NPASS; j++) {
            if (KS * j >= nt) break;
            const int idx = KS * j + kk, key = t0 + idx;
            float ks = F16 ? 1.f : h2f(ksr[j]);
            if (sp.has_new && key == sp.pq) {
                if constexpr (F16) {
#pragma unroll
                    for (int c = 0; c < NQ / 2; c++) kr[j].w[c] = *(const uint32_t *)(S.new16[0] + qq * NQ + 2 * c);
                } else {
#pragma unroll
                    for (int c = 0; c < NQ / 4; c++) kr[j].w[c] = *(const uint32_t *)(S.new8[0] + qq * NQ + 4 * c);
                    ks = h2f(S.new_sc[0][(qq * NQ) / 32]);
                }
            }
            float acc[G];
#pragma unroll
            for (int g = 0; g < G; g++) acc[g] = 0.f;
#pragma unroll
            for (int e4 = 0; e4 < NQ / 4; e4++) {
                float kf[4];
#pragma unroll
                for (int i = 0; i < 4; i++) kf[i] = kv_value<F16>(kr[j].w, 4 * e4 + i) * ks;
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const float4 qv = *(const float4 *)&S.q_s[g][qq * NQ + 4 * e4];
                    acc[g] += qv.x * kf[0] + qv.y * kf[1] + qv.z * kf[2] + qv.w * kf[3];
                }
            }
#pragma unroll
            for (int g = 0; g < G; g++) {
                acc[g] = dpp_add<0xB1, 0xF, true>(acc[g]);  // quad_perm [1,0,3,2]
                acc[g] = dpp_add<0x4E, 0xF, true>(acc[g]);  // quad_perm [2,3,0,1]
            }
            if (qq == 0) {
#pragma unroll
                for (int g = 0; g < G; g++) S.p_s[idx][g] = idx < nt ? acc[g] * a.scale : -INFINITY;
            }
        }
        __syncthreads();
        // Online softmax per head over the pass.
        for (int g = wave; g < G; g += NT / 64) {
            float v[SMX];
            float mt = -INFINITY;
#pragma unroll
            for (int i = 0; i < SMX; i++) {
                v[i] = 64 * i + lane < nt ? S.p_s[64 * i + lane][g] : -INFINITY;
                mt = fmaxf(mt, v[i]);
            }
            mt = wave_max_dpp(mt);
            const float mo = S.m_s[g], mn = fmaxf(mo, mt);
            float ls = 0.f;
#pragma unroll
            for (int i = 0; i < SMX; i++) {
                const float pe = v[i] == -INFINITY ? 0.f : expf(v[i] - mn);
                if (64 * i < nt) S.p_s[64 * i + lane][g] = pe;
                ls += pe;
            }
            ls = wave_sum_dpp(ls);
            if (lane == 0) {
                const float al = mo == -INFINITY ? 0.f : expf(mo - mn);
                S.alpha_s[g] = al;
                S.m_s[g] = mn;
                S.l_s[g] = S.l_s[g] * al + ls;
            }
        }
        __syncthreads();
        // o = o * alpha + sum over the pass's keys of p * v.
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float al = S.alpha_s[g];
#pragma unroll
            for (int e = 0; e < 8; e++) o[g][e] *= al;
        }
#pragma unroll
        for (int s2 = 0; s2 < NVS; s2++) {
            if (s2 * KPS >= nt) break;
            const int idx = s2 * KPS + wave * KPW + vk, key = t0 + idx;
            VRow<F16> v8 = vr[s2];
            float vs = F16 ? 1.f : h2f(vsr[s2]);
            if (sp.has_new && key == sp.pq) {
                if constexpr (F16) {
                    v8 = *(const VRow<F16> *)(S.new16[1] + 8 * vc);
                } else {
                    v8 = *(const VRow<F16> *)(S.new8[1] + 8 * vc);
                    vs = h2f(S.new_sc[1][(8 * vc) / 32]);
                }
            }
            float w[G];
#pragma unroll
            for (int g = 0; g < G; g++) w[g] = S.p_s[idx][g] * vs;  // idx < 64 * ceil(nt / 64): a written row
            const uint32_t *vw = (const uint32_t *)&v8;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const float vf = kv_value<F16>(vw, e);
#pragma unroll
                for (int g = 0; g < G; g++) o[g][e] += w[g] * vf;
            }
        }
        __syncthreads();  // p_s is rewritten by the next pass
    }
    // The wave's KPW key groups of the same dims (lanes i ^ 8, ^ 16, ^ 32),
    // then the 4 waves.
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
            float v = o[g][e];
            if constexpr (LPV <= 8) v = dpp_add<0x128, 0xF, true>(v);  // row_ror:8 within 16-lane rows
            if constexpr (LPV <= 16) v = add_xor16(v);
            o[g][e] = add_xor32(v);
        }
    if (vk == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            *(float4 *)&S.o_s[wave][g * HD + 8 * vc] = make_float4(o[g][0], o[g][1], o[g][2], o[g][3]);
            *(float4 *)&S.o_s[wave][g * HD + 8 * vc + 4] = make_float4(o[g][4], o[g][5], o[g][6], o[g][7]);
        }
    }
    __syncthreads();

    constexpr int64_t rec = HD + 2, grp = attn_group_floats(G, HD);
    float *pb = a.part + (((int64_t)b * n_split + split) * a.HKV + kvh) * grp;
    for (int j = tid; j < G * HD; j += NT) {
        const int g = j / HD, d = j % HD;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) v += S.o_s[w][j];
        st_dev(pb + g * rec + d, v);
    }
    if (tid < G) {
        st_dev(pb + tid * rec + HD, S.m_s[tid]);
        st_dev(pb + tid * rec + HD + 1, S.l_s[tid]);
    }
    wait_stores();
    __syncthreads();
    if (tid == 0) S.last = atomicAdd(a.counters + (b * a.HKV + kvh) * CTR_STRIDE, 1) == n_split - 1;
    __syncthreads();
    if (!S.last) return;
    // The merge: this thread's outputs of every split (up to 32 at a time)
    // and every split's (m, l) are requested together; a wave per head turns
    // the (m, l) into weights, a lane per split.
    const float *p_all = a.part + ((int64_t)b * n_split * a.HKV + kvh) * grp;
    const int64_t sstride = (int64_t)a.HKV * grp;
    constexpr int OPT = (G * HD + NT - 1) / NT, MC = 32;
    float acc[OPT];
#pragma unroll
    for (int k = 0; k < OPT; k++) acc[k] = 0.f;
    for (int s0 = 0; s0 < n_split; s0 += MC) {
        const int nc = min(MC, n_split - s0);
        float ov[OPT][MC];
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            const int j = min(tid + NT * k, G * HD - 1), g = j / HD, d = j % HD;
#pragma unroll
            for (int i = 0; i < MC; i++) ov[k][i] = ld_dev(p_all + (int64_t)(s0 + min(i, nc - 1)) * sstride + g * rec + d);
        }
        if (s0 == 0) {
            for (int g = wave; g < G; g += NT / 64) {
                const int sl = min(lane, n_split - 1);
                const float m0 = ld_dev(p_all + (int64_t)sl * sstride + g * rec + HD);
                const float l0 = ld_dev(p_all + (int64_t)sl * sstride + g * rec + HD + 1);
                const float m = lane < n_split ? m0 : -INFINITY;
                const float M = wave_max_dpp(m);
                const float w = m == -INFINITY ? 0.f : expf(m - M);
                const float L = wave_sum_dpp(w * (lane < n_split ? l0 : 0.f));
                S.wts[g][lane] = w;  // lanes past n_split: 0
                if (lane == 0) S.red[g] = L;
            }
            __syncthreads();
        }
#pragma unroll
        for (int k = 0; k < OPT; k++) {
            const int j = min(tid + NT * k, G * HD - 1), g = j / HD;
            float v = acc[k];
#pragma unroll
            for (int i4 = 0; i4 < MC / 4; i4++) {  // weights past n_split are 0 (their o: a valid split's)
                const float4 w = *(const float4 *)&S.wts[g][s0 + 4 * i4];
                v += w.x * ov[k][4 * i4] + w.y * ov[k][4 * i4 + 1] + w.z * ov[k][4 * i4 + 2] + w.w * ov[k][4 * i4 + 3];
            }
            acc[k] = v;
        }
    }
#pragma unroll
    for (int k = 0; k < OPT; k++) {
        const int j = tid + NT * k;
        if (j < G * HD) {
            const int g = j / HD, d = j % HD;
            st_dev(a.out + (int64_t)b * a.H * HD + (int64_t)(kvh * G + g) * HD + d, acc[k] / S.red[g]);
        }
    }
    if (tid == 0) st_dev(a.counters + (b * a.HKV + kvh) * CTR_STRIDE, 0);  // ready for the next use
}

}  // namespace ts5hip
