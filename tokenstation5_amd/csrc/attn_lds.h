// Device core of the short-slice decode attention (k_attn_lds in
// attention.hip): one query whose work items hold at most a few hundred keys
// (a cache of up to 8192 positions), where the work item shares its slice's
// scores, softmax and p * v through LDS across all its lanes, which is faster
// there than the per-wave key loop of attn_core.h.
#pragma once
#include "attn_core.h"

namespace ts5hip {

// K bytes per lane of a key's score: NQ = HD / (NT / 64) lanes' worth.
template <int NQ>
struct LdsKRow {
    uint32_t w[NQ / 4];
};
template <int NQ>
__device__ inline LdsKRow<NQ> lds_load_krow(const int8_t *p) {
    LdsKRow<NQ> r;
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

// ---------------------------------------------------------------------------
// One work item (split, KV head kvh, query b) of n_split over its whole key
// slice, in passes of up to LDS_KT keys: the query's inputs are requested
// first, then every K and V byte of a pass, held in registers while the
// query is prepared, so the slice costs one memory round trip rather than
// one per 64-key tile.
//   scores   4 lanes per key (HD/4 dims each), 64 keys per sweep of the
//            workgroup, q from LDS, the 4 partial sums added by DPP;
//   softmax  a wave per head over the pass, online across passes;
//   p * v    8 dims per lane straight from the V rows in registers, G heads
//            per V value; the lanes and waves that took other keys of the
//            same dims are added at the end (shuffles, then LDS).
// Then the partial record [G x (HD values, m, l)] and the merge.
// ---------------------------------------------------------------------------
constexpr int LDS_KT = 256;

template <int HD, int G, int NT = 256>
struct LdsSliceLds {
    float q_s[G][HD];
    __align__(16) float p_s[LDS_KT][G];  // scores, then probabilities
    float alpha_s[G], m_s[G], l_s[G], red[G];
    float kv_s[1][2][HD];                    // the new token's K and V before rounding (one query: one new key)
    __align__(16) int8_t new8[1][2][HD];     // ... and after, as int8
    uint16_t new_sc[1][2][HD / 32];          // ... with their f16 scales
    __align__(16) uint16_t new16[1][2][HD];  // ... or as f16 (an f16 cache)
    __align__(16) float o_s[NT / 64][G * HD];  // each wave's p * v sums
    __align__(16) float wts[G][ATTN_MAX_SPLIT];  // the merge's weight per (head, split), 0 past n_split
    int last;
};

template <int HD, int G, int NT>
struct LdsSliceShape {
    // Scores: LPK lanes a key, KS keys a sweep of the workgroup, NPASS sweeps a
    // pass. p * v: DPL dims a lane, KPW keys a wave, KPS keys a step, NVS steps.
    static constexpr int NW = NT / 64, LPK = 4, NQ = HD / LPK, KS = NT / LPK, NPASS = LDS_KT / KS;
    static constexpr int DPL = 8, LPV = HD / DPL, KPW = 64 / LPV, KPS = NW * KPW, NVS = LDS_KT / KPS;
    static_assert(NQ % 8 == 0 && LPV <= 64 && 64 % LPV == 0 && 64 % KPS == 0 && LDS_KT % KS == 0,
                  "attention slice shape");
};

// The cache's values: q8 (int8 with an f16 scale per 32) or, with F16, f16
// (2 bytes a value, no scales; ks / vs unused). A lane's 8 V dims are one
// uint2 of int8 or one uint4 of f16.
template <bool F16>
using LdsVRow = typename std::conditional<F16, uint4, uint2>::type;
template <int HD, int G, int NT, bool F16 = false>
__device__ inline void attn_slice_lds(const AttnArgs &a, int split, int kvh, int b, int n_split,
                                  LdsSliceLds<HD, G, NT> &S) {
    using SH = LdsSliceShape<HD, G, NT>;
    constexpr int NW = SH::NW, NQ = SH::NQ, KS = SH::KS, NPASS = SH::NPASS, LPV = SH::LPV, KPW = SH::KPW,
                  KPS = SH::KPS, NVS = SH::NVS, SMX = LDS_KT / 64;
    constexpr int VB = F16 ? 2 : 1;  // bytes per cached value
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kk = tid >> 2, qq = tid & 3;              // scores: key kk of a sweep, quarter qq of the dims
    const int vk = lane / LPV, vc = lane % LPV;         // p * v: key vk of a wave's step, dims 8 vc ..
    const AttnSpan sp = attn_span<16>(a, split, kvh, b, n_split);
    if (split >= sp.used) return;  // an empty split: not counted, not merged
    const int8_t *kb = a.kv.k + sp.head_base * HD * VB, *vb = a.kv.v + sp.head_base * HD * VB;
    const uint16_t *ksb = F16 ? nullptr : a.kv.ks + sp.head_base * (HD / 32);
    const uint16_t *vsb = F16 ? nullptr : a.kv.vs + sp.head_base * (HD / 32);
    float o[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < 8; e++) o[g][e] = 0.f;
    // The query's (and its new key's) inputs are requested first: loads
    // complete in order, so the preparation then runs while the slice's K/V
    // (requested next) are still arriving.
    AttnPre<HD, G, NT> pre;
    attn_preload<HD, G, NT>(a, kvh, b, sp, pre);
    bool prepared = false;
    for (int t0 = sp.p0; t0 < sp.p1 || !prepared; t0 += LDS_KT) {
        const int nt = max(0, min(LDS_KT, sp.p1 - t0));
        const int kmax = max(sp.p1 - 1, 0);  // loads past the slice read its last key (zero weight)
        LdsKRow<NQ * VB> kr[NPASS];
        uint16_t ksr[NPASS];
#pragma unroll
        for (int j = 0; j < NPASS; j++) {
            const int key = min(t0 + KS * j + kk, kmax);
            kr[j] = lds_load_krow<NQ * VB>(kb + ((int64_t)key * HD + qq * NQ) * VB);
            if constexpr (!F16) ksr[j] = ksb[(int64_t)key * (HD / 32) + (qq * NQ) / 32];
        }
        LdsVRow<F16> vr[NVS];
        uint16_t vsr[NVS];
#pragma unroll
        for (int s2 = 0; s2 < NVS; s2++) {
            const int key = min(t0 + s2 * KPS + wave * KPW + vk, kmax);
            vr[s2] = *(const LdsVRow<F16> *)(vb + ((int64_t)key * HD + 8 * vc) * VB);
            if constexpr (!F16) vsr[s2] = vsb[(int64_t)key * (HD / 32) + (8 * vc) / 32];
        }
        if (!prepared) {
            attn_prepare<HD, G, NT, F16>(a, kvh, b, sp, S, &pre);
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
                    for (int c = 0; c < NQ / 2; c++) kr[j].w[c] = *(const uint32_t *)(S.new16[0][0] + qq * NQ + 2 * c);
                } else {
#pragma unroll
                    for (int c = 0; c < NQ / 4; c++) kr[j].w[c] = *(const uint32_t *)(S.new8[0][0] + qq * NQ + 4 * c);
                    ks = h2f(S.new_sc[0][0][(qq * NQ) / 32]);
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
            LdsVRow<F16> v8 = vr[s2];
            float vs = F16 ? 1.f : h2f(vsr[s2]);
            if (sp.has_new && key == sp.pq) {
                if constexpr (F16) {
                    v8 = *(const LdsVRow<F16> *)(S.new16[0][1] + 8 * vc);
                } else {
                    v8 = *(const LdsVRow<F16> *)(S.new8[0][1] + 8 * vc);
                    vs = h2f(S.new_sc[0][1][(8 * vc) / 32]);
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

    if (sp.used == 1) {  // the only split with keys (a short cache): the output directly, as the merge would
        for (int q = tid; q < G * HD / 4; q += NT) {
            float4 v = *(const float4 *)&S.o_s[0][4 * q];
#pragma unroll
            for (int w = 1; w < NW; w++) {
                const float4 o = *(const float4 *)&S.o_s[w][4 * q];
                v.x += o.x, v.y += o.y, v.z += o.z, v.w += o.w;
            }
            const float L = S.l_s[4 * q / HD];
            const float4 r = L > 0.f ? make_float4(v.x / L, v.y / L, v.z / L, v.w / L) : make_float4(0.f, 0.f, 0.f, 0.f);
            *(float4 *)(a.out + (int64_t)b * a.H * HD + (int64_t)kvh * G * HD + 4 * q) = r;
        }
        return;
    }
    attn_publish<G, HD, NT>(
        attn_part_group<G, HD>(a, b, split, kvh, n_split),
        [&](int q) {
            float4 v = *(const float4 *)&S.o_s[0][4 * q];
#pragma unroll
            for (int w = 1; w < NW; w++) {
                const float4 o = *(const float4 *)&S.o_s[w][4 * q];
                v.x += o.x, v.y += o.y, v.z += o.z, v.w += o.w;
            }
            return v;
        },
        [&](int g) { return make_float2(S.m_s[g], S.l_s[g]); });
    __syncthreads();
    if (tid == 0) S.last = atomicAdd(a.counters + (b * a.HKV + kvh) * CTR_STRIDE, 1) == sp.used - 1;
    __syncthreads();
    if (!S.last) return;
    attn_merge<G, HD, NT>(a, b, kvh, n_split, sp.used, S.wts, S.red, &S.o_s[0][0]);
}

}  // namespace ts5hip
