// Split-K attention of a batch of consecutive queries over one q8 cache on
// the matrix cores (a verify batch: the pending token and its drafts), used
// by attention.hip for B x G <= 32 rows of head dimension 128. The same
// arithmetic as the decode kernel (engine/src/cpu_backend.cpp:224-248 per
// query; merge attn_merge.comp:18-47), with every query of the batch in one
// work item, so that each key is read and converted once for all of them.
//
// Grid (n_split, HKV), 8 waves (two sets of 4, 16 rows each). Row r = G b + g is head g of KV head kvh
// for token b (position n0 + b, keys [0, n0 + b]); rows B G .. 31 are empty.
//  1. Preparation: the rows' queries (bias, per-head norm, RoPE when `rope`)
//     into LDS; with `append`, the batch's new keys in this key slice (K with
//     RoPE at its own position, V) rounded to q8 and stored at their cache
//     slots, then read back with the slice like every other key.
//  2. Each wave of a set takes 16 keys of every 64-key step of the slice:
//     S^T (16 keys x 32 rows) = K . Q^T on v_mfma_f32_16x16x32_f16 per
//     32-value scale group: K as exact fp16 integers, the rows as fp16 hi +
//     lo planes of q * scale * log2(e) * 2^-e (e per row), then S += ks * R;
//     online softmax per row in the log2 domain (rows are the lanes' columns);
//     O^T (128 dims x 32 rows) += V^T . (P o vs)^T on v_mfma_f32_16x16x16_f16:
//     V as exact fp16 v8 / 128, transposed through the wave's own LDS, and
//     P scaled by 128 times each key's V scale of the dims' group, as fp16
//     hi + lo (B operand layout = the D layout of S^T: P never leaves
//     registers).
//  3. The waves' (m, l, O) combine in LDS into the work item's partial;
//     a second launch (a workgroup per row and KV head) merges the splits'
//     partials in split order: O = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s,
//     and can write the output as the next matmul's activation records too.
#pragma once
#include "attn_core.h"

namespace ts5hip {

typedef _Float16 mq_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 mq_h4 __attribute__((ext_vector_type(4)));
typedef _Float16 mq_h2 __attribute__((ext_vector_type(2)));
typedef float mq_f4 __attribute__((ext_vector_type(4)));

constexpr int MQ_HD = 128;
constexpr int MQ_ROWS = 32;           // two 16-row MFMA tiles
constexpr int MQ_QT = 1;              // 16-row tiles a wave (the rows of a wave set)
constexpr int MQ_KG = 4;              // waves of a set, each 16 keys of a step
constexpr int MQ_NW = MQ_KG * (MQ_ROWS / 16 / MQ_QT), MQ_NT = 64 * MQ_NW;
constexpr int MQ_WR = 16 * MQ_QT;     // rows a wave
constexpr int MQ_STEP = 16 * MQ_KG;   // keys of a workgroup step
constexpr int MQ_REC = MQ_HD + 4;     // partial record: m, l, -, -, O[128]
constexpr int MQ_VT = 10;             // dwords per dim of a wave's V^T (4 key quads + padding)

struct MqLds {
    union {
        struct {
            float q_s[MQ_ROWS][MQ_HD];             // the rows' queries, prepared
            float kv_s[ATTN_MAX_NEW][2][MQ_HD];    // the slice's new keys before rounding
        };
        __align__(16) float o_w[MQ_NW][MQ_WR][MQ_REC];  // each wave's O rows, after the keys
    };
    __align__(16) uint32_t vt[MQ_NW][MQ_HD * MQ_VT];  // each wave's 16 keys' V^T, [d][key quad] as f16
    float m_w[MQ_NW][MQ_WR], l_w[MQ_NW][MQ_WR];
};

// 8 int8 -> 8 exact fp16: 0x64xx is 1024 + xx, so (b + 128) in the low byte
// gives 1152 + b.
__device__ inline mq_h8 mq_i8x8(uint32_t w0, uint32_t w1) {
    const mq_h2 k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
    const uint32_t v0 = w0 ^ 0x80808080u, v1 = w1 ^ 0x80808080u;
    mq_h2 h[4];
    h[0] = __builtin_bit_cast(mq_h2, __builtin_amdgcn_perm(0x64646464u, v0, 0x04010400u)) - k1152;
    h[1] = __builtin_bit_cast(mq_h2, __builtin_amdgcn_perm(0x64646464u, v0, 0x04030402u)) - k1152;
    h[2] = __builtin_bit_cast(mq_h2, __builtin_amdgcn_perm(0x64646464u, v1, 0x04010400u)) - k1152;
    h[3] = __builtin_bit_cast(mq_h2, __builtin_amdgcn_perm(0x64646464u, v1, 0x04030402u)) - k1152;
    return mq_h8{h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
}

// 1. Queries of the R rows into q_s (rows past R zero); the new keys of the
// slice [nlo, nhi) rounded to q8 and stored at their cache slots (this work
// item is the only one whose slice holds them), the stores complete before
// the final barrier so that the slice's loads after it read them. Every
// global load (rows, bias, new keys, RoPE table entries) is requested before
// the first is used.
__device__ inline void mq_prepare(const AttnArgs &a, int kvh, int G, int B, int n0, int p0, int p1, MqLds &S) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int R = B * G;
    const int nlo = max(n0, p0), nhi = a.append ? min(n0 + B, p1) : nlo, nn = max(nhi - nlo, 0);
    constexpr int F4 = MQ_HD / 4;                       // float4s a row
    constexpr int QK = MQ_ROWS * F4 / MQ_NT;            // query float4s a thread
    constexpr int KK = ATTN_MAX_NEW * 2 * F4 / MQ_NT;   // new-key float4s a thread
    constexpr int QP = MQ_ROWS * (MQ_HD / 2) / MQ_NT;   // query RoPE pairs a thread
    constexpr int KP = ATTN_MAX_NEW * (MQ_HD / 2) / MQ_NT;  // key RoPE pairs a thread
    static_assert(QK * MQ_NT == MQ_ROWS * F4 && KK * MQ_NT == ATTN_MAX_NEW * 2 * F4, "whole rows a pass");
    const int nr2 = a.n_rot / 2;
    float4 qv[QK], kv[KK];
    float2 qcs[QP], kcs[KP];
#pragma unroll
    for (int k = 0; k < QK; k++) {
        const int f = tid + MQ_NT * k, r = f / F4, d = 4 * (f % F4);
        qv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < R) {
            const int64_t e = (int64_t)(kvh * G + r % G) * MQ_HD + d;
            qv[k] = *(const float4 *)(a.q + (int64_t)(r / G) * a.q_stride + e);
            if (a.rope && a.bias) {
                const float4 bv = *(const float4 *)(a.bias + e);
                qv[k].x += bv.x, qv[k].y += bv.y, qv[k].z += bv.z, qv[k].w += bv.w;
            }
        }
    }
#pragma unroll
    for (int k = 0; k < KK; k++) {
        const int f = tid + MQ_NT * k, kk = f / (2 * F4), which = (f / F4) & 1, d = 4 * (f % F4);
        kv[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (kk < nn) {
            const int64_t e = (int64_t)((which ? a.H + a.HKV : a.H) + kvh) * MQ_HD + d;
            kv[k] = *(const float4 *)(a.q + (int64_t)(nlo + kk - n0) * a.q_stride + e);  // the token at that position
            if (a.bias) {
                const float4 bv = *(const float4 *)(a.bias + e);
                kv[k].x += bv.x, kv[k].y += bv.y, kv[k].z += bv.z, kv[k].w += bv.w;
            }
        }
    }
    if (a.rope) {
#pragma unroll
        for (int k = 0; k < QP; k++) {
            const int j = tid + MQ_NT * k, r = j / (MQ_HD / 2), i = j % (MQ_HD / 2);
            qcs[k] = r < R && i < nr2 ? a.rope_cs[(int64_t)(n0 + r / G) * nr2 + i] : make_float2(1.f, 0.f);
        }
#pragma unroll
        for (int k = 0; k < KP; k++) {
            const int j = tid + MQ_NT * k, kk = j / (MQ_HD / 2), i = j % (MQ_HD / 2);
            kcs[k] = kk < nn && i < nr2 ? a.rope_cs[(int64_t)(nlo + kk) * nr2 + i] : make_float2(1.f, 0.f);
        }
    }
#pragma unroll
    for (int k = 0; k < QK; k++) {
        const int f = tid + MQ_NT * k;
        *(float4 *)&S.q_s[f / F4][4 * (f % F4)] = qv[k];
    }
#pragma unroll
    for (int k = 0; k < KK; k++) {
        const int f = tid + MQ_NT * k, kk = f / (2 * F4), which = (f / F4) & 1;
        if (kk < nn) *(float4 *)&S.kv_s[kk][which][4 * (f % F4)] = kv[k];
    }
    __syncthreads();
    if (a.rope) {
        if (a.q_norm || (nn && a.k_norm)) {  // qwen3's per-head q_norm / k_norm
            for (int g = wave; g < R + nn; g += MQ_NW) {
                const float *nw = g < R ? a.q_norm : a.k_norm;
                if (!nw) continue;
                float *v = g < R ? S.q_s[g] : S.kv_s[g - R][0];
                float ss = 0.f;
                for (int j = lane; j < MQ_HD; j += 64) ss += v[j] * v[j];
                ss = wave_sum(ss);
                const float sc = 1.0f / sqrtf(ss / (float)MQ_HD + a.eps);
                for (int j = lane; j < MQ_HD; j += 64) v[j] = v[j] * sc * nw[j];
            }
            __syncthreads();
        }
        // The query heads at their tokens' positions, each key at its own
        // (x0 c - x1 s, x0 s + x1 c with separate roundings).
#pragma unroll
        for (int k = 0; k < QP; k++) {
            const int j = tid + MQ_NT * k, r = j / (MQ_HD / 2), i = j % (MQ_HD / 2);
            if (r < R && i < nr2) {
                float *v = S.q_s[r];
                const int i0 = a.neox ? i : 2 * i, i1 = a.neox ? i + nr2 : 2 * i + 1;
                float x0 = v[i0], x1 = v[i1];
                rope_pair(x0, x1, qcs[k].x, qcs[k].y);
                v[i0] = x0, v[i1] = x1;
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < KP; k++) {
            const int j = tid + MQ_NT * k, kk = j / (MQ_HD / 2), i = j % (MQ_HD / 2);
            if (kk < nn && i < nr2) {
                float *v = S.kv_s[kk][0];
                const int i0 = a.neox ? i : 2 * i, i1 = a.neox ? i + nr2 : 2 * i + 1;
                float x0 = v[i0], x1 = v[i1];
                rope_pair(x0, x1, kcs[k].x, kcs[k].y);
                v[i0] = x0, v[i1] = x1;
            }
        }
        __syncthreads();
    }
    if (nn == 0) return;
    // q8 (engine/src/cpu_backend.cpp:78-90): per 32 values sc = f16(amax / 127),
    // q = clamp(rint(v / sc), +-127); a wave per (key, K or V), two values a lane.
    for (int pr = wave; pr < 2 * nn; pr += MQ_NW) {
        const int kk = pr >> 1, which = pr & 1, i = lane;
        const int64_t slot = (int64_t)kvh * a.n_ctx + nlo + kk;
        const float a0 = S.kv_s[kk][which][2 * i], a1 = S.kv_s[kk][which][2 * i + 1];
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
        *(uint16_t *)((which ? a.kv.v : a.kv.k) + slot * MQ_HD + 2 * i) = (uint16_t)((q0 & 0xff) | ((q1 & 0xff) << 8));
        if ((i & 15) == 0) (which ? a.kv.vs : a.kv.ks)[slot * (MQ_HD / 32) + i / 16] = sh;
    }
    wait_stores();
    __syncthreads();
}

__device__ inline void attn_mq(const AttnArgs &a, int G, int B, int split, int kvh, int n_split, MqLds &S) {
    constexpr float LOG2E = 1.4426950408889634f;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rl = lane & 15, kq = lane >> 4;
    const int kg = wave % MQ_KG, rbase = (wave / MQ_KG) * MQ_WR;  // the wave's keys of a step, its first row
    const int R = B * G;
    const int n0 = a.n_keys[0], nk = n0 + B;  // the last query reads keys [0, nk)
    int chunk = (nk + n_split - 1) / n_split;
    chunk = (chunk + MQ_STEP - 1) / MQ_STEP * MQ_STEP;
    const int used = (nk + chunk - 1) / chunk;
    if (split >= used) return;  // an empty split: not counted, not merged
    const int p0 = split * chunk, p1 = min(nk, p0 + chunk), nkeys = p1 - p0;
    // The slice's K and V (and scales) as bounded buffers from key p0: past
    // p1 they read zeros and touch no memory.
    const int64_t base = (int64_t)kvh * a.n_ctx + p0;
    const __amdgpu_buffer_rsrc_t rk = slice_rsrc(a.kv.k + base * MQ_HD, (uint32_t)nkeys * MQ_HD);
    const __amdgpu_buffer_rsrc_t rv = slice_rsrc(a.kv.v + base * MQ_HD, (uint32_t)nkeys * MQ_HD);
    const __amdgpu_buffer_rsrc_t rks = slice_rsrc(a.kv.ks + base * 4, (uint32_t)nkeys * 8);
    const __amdgpu_buffer_rsrc_t rvs = slice_rsrc(a.kv.vs + base * 4, (uint32_t)nkeys * 8);
    // A step's loads for this wave's 16 keys kl .. kl + 15 (relative to p0):
    // K: key kl + rl, dims 32 c + 8 kq .. + 7 (the A operand of group c);
    // V: keys kl + 4 kq + i, dims 8 rl .. 8 rl + 7 (the lane's share of the
    // transpose); the K and V scales of keys kl + 4 kq + i (the lane's S and
    // P entries), all 4 groups.
    struct Step {
        u32x2 k[4], v[4];
        u32x4 ks[2], vs[2];
    };
    auto load = [&](Step &w, int st) {
        const uint32_t kl = (uint32_t)(st * MQ_STEP + kg * 16);
#pragma unroll
        for (int c = 0; c < 4; c++) w.k[c] = __builtin_amdgcn_raw_buffer_load_b64(rk, (kl + rl) * MQ_HD + 32 * c + 8 * kq, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) w.v[i] = __builtin_amdgcn_raw_buffer_load_b64(rv, (kl + 4 * kq + i) * MQ_HD + 8 * rl, 0, 0);
#pragma unroll
        for (int h = 0; h < 2; h++) {
            w.ks[h] = __builtin_amdgcn_raw_buffer_load_b128(rks, (kl + 4 * kq) * 8 + 16 * h, 0, 0);
            w.vs[h] = __builtin_amdgcn_raw_buffer_load_b128(rvs, (kl + 4 * kq) * 8 + 16 * h, 0, 0);
        }
    };
    // The first two steps' loads go out before the preparation, except
    // where the slice holds new keys: those are read after their stores.
    const bool fresh = a.append && p1 > n0;
    Step A, Bs;
    if (!fresh) load(A, 0), load(Bs, 1);
    mq_prepare(a, kvh, G, B, n0, p0, p1, S);

    if (fresh) load(A, 0), load(Bs, 1);
    // The lane's rows (its MFMA columns) rbase + 16 qt + rl as B operands:
    // dims 32 c + 8 kq .. + 7 of q * scale * log2(e) * 2^-e, hi and lo.
    mq_h8 qh[MQ_QT][4], ql[MQ_QT][4];
    float p2e[MQ_QT];
    int pos[MQ_QT];
#pragma unroll
    for (int qt = 0; qt < MQ_QT; qt++) {
        const int r = rbase + 16 * qt + rl;
        pos[qt] = r < R ? n0 + r / G : -1;  // empty rows take no key
        float v[4][8], amax = 0.f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float4 x0 = *(const float4 *)&S.q_s[r][32 * c + 8 * kq];
            const float4 x1 = *(const float4 *)&S.q_s[r][32 * c + 8 * kq + 4];
            const float f[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) v[c][j] = f[j] * (a.scale * LOG2E), amax = fmaxf(amax, fabsf(v[c][j]));
        }
        amax = max_xor32(max_xor16(amax));
        const int e = amax > 0.f ? max(ilogbf(amax) - 13, -100) : 0;
        const float sc = ldexpf(1.0f, -e);
        p2e[qt] = ldexpf(1.0f, e);
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float f = v[c][j] * sc;  // exact: sc is a power of 2
                qh[qt][c][j] = (_Float16)f;
                ql[qt][c][j] = (_Float16)(f - (float)qh[qt][c][j]);
            }
    }

    mq_f4 O[MQ_QT][8];
    float m[MQ_QT], l[MQ_QT];
#pragma unroll
    for (int qt = 0; qt < MQ_QT; qt++) {
        m[qt] = -INFINITY, l[qt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < 8; dt++) O[qt][dt] = mq_f4{0.f, 0.f, 0.f, 0.f};
    }
    uint32_t *vt = S.vt[wave];
    auto step = [&](const Step &w, int st) {
        const int kl = st * MQ_STEP + kg * 16;
        // Scales: halfword 4 i + c of the pair of u32x4 is key kl + 4 kq + i, group c.
        float ksf[4][4], vsf[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int hw = 4 * i + c;
                ksf[i][c] = h2f((w.ks[hw >> 3][(hw >> 1) & 3] >> (16 * (hw & 1))) & 0xffff);
                vsf[i][c] = 128.f * h2f((w.vs[hw >> 3][(hw >> 1) & 3] >> (16 * (hw & 1))) & 0xffff);
            }
        // S^T: D[key 4 kq + i][row rbase + 16 qt + rl].
        float s[MQ_QT][4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const mq_h8 ka = mq_i8x8(w.k[c][0], w.k[c][1]);
#pragma unroll
            for (int qt = 0; qt < MQ_QT; qt++) {
                mq_f4 Rr = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[qt][c], mq_f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                Rr = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[qt][c], Rr, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) s[qt][i] = c == 0 ? ksf[i][c] * Rr[i] : fmaf(ksf[i][c], Rr[i], s[qt][i]);
            }
        }
        // V^T of the wave's 16 keys into its LDS: dim d = 8 rl + j, key quad
        // kq (keys 4 kq + i) as 4 f16 at dword 10 d + 2 kq, each value
        // v8 / 128 (exact; P carries the 128, which keeps the lo plane of
        // p * vs * 128 out of the f16 subnormals for all but tiny p).
        {
            const mq_h8 k2m7 = {(_Float16)0.0078125f, (_Float16)0.0078125f, (_Float16)0.0078125f,
                                (_Float16)0.0078125f, (_Float16)0.0078125f, (_Float16)0.0078125f,
                                (_Float16)0.0078125f, (_Float16)0.0078125f};
            mq_h8 hv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) hv[i] = mq_i8x8(w.v[i][0], w.v[i][1]) * k2m7;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const mq_h4 col = {hv[0][j], hv[1][j], hv[2][j], hv[3][j]};
                *(mq_h4 *)&vt[(8 * rl + j) * MQ_VT + 2 * kq] = col;
            }
        }
        // Online softmax per row (log2 domain), then the B operands
        // (P o vs of group g) as hi + lo.
        mq_h4 ph[MQ_QT][4], pl[MQ_QT][4];
#pragma unroll
        for (int qt = 0; qt < MQ_QT; qt++) {
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = p0 + kl + 4 * kq + i;
                const float sv = key < p1 && key <= pos[qt] ? s[qt][i] * p2e[qt] : -INFINITY;
                s[qt][i] = sv;
                mx = fmaxf(mx, sv);
            }
            mx = max_xor32(max_xor16(mx));
            const float mn = fmaxf(m[qt], mx);
            const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f(m[qt] - mn);
            float p[4], sum = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                p[i] = mn == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s[qt][i] - mn);
                sum += p[i];
            }
            sum = add_xor32(add_xor16(sum));
            m[qt] = mn, l[qt] = l[qt] * alpha + sum;
            if (alpha != 1.0f) {
#pragma unroll
                for (int dt = 0; dt < 8; dt++) O[qt][dt] *= alpha;
            }
            // x = p * vs rounded to fp32 before its split: the empty asm keeps
            // the product out of the conversions (contracted, hi would be
            // rounded from the exact product and lo from the rounded one, or
            // the other way round, one f16 ulp apart at a rounding midpoint),
            // so that hi + lo is x.
#pragma unroll
            for (int g = 0; g < 4; g++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    float x = p[i] * vsf[i][g];
                    asm volatile("" : "+v"(x));
                    ph[qt][g][i] = (_Float16)x;
                    pl[qt][g][i] = (_Float16)(x - (float)ph[qt][g][i]);
                }
        }
        // O^T += V^T (P o vs)^T: A = V^T rows 16 dt + rl, keys 4 kq .. + 3
        // (the wave's own LDS writes above are in: one wave, in order).
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const mq_h4 va = *(const mq_h4 *)&vt[(16 * dt + rl) * MQ_VT + 2 * kq];
#pragma unroll
            for (int qt = 0; qt < MQ_QT; qt++) {
                O[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, ph[qt][dt >> 1], O[qt][dt], 0, 0, 0);
                O[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl[qt][dt >> 1], O[qt][dt], 0, 0, 0);
            }
        }
        // The next step's V^T writes must not pass these reads: in order.
    };
    // Two register sets in turn; each is refilled with the step two on as
    // soon as it is used (past the slice: no memory access).
    const int nsteps = (nkeys + MQ_STEP - 1) / MQ_STEP;
    for (int st = 0; st < nsteps; st += 2) {
        step(A, st);
        if (st + 1 >= nsteps) break;
        load(A, st + 2);
        step(Bs, st + 1);
        load(Bs, st + 3);
    }
    __syncthreads();  // every wave is past its reads of q_s: o_w overlays it

    // The waves' rows: O^T[d = 16 dt + 4 kq + i][row rbase + 16 qt + rl], at
    // the wave's local row 16 qt + rl.
#pragma unroll
    for (int qt = 0; qt < MQ_QT; qt++) {
        const int r = 16 * qt + rl;
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
            *(float4 *)&S.o_w[wave][r][4 + 16 * dt + 4 * kq] = make_float4(O[qt][dt][0], O[qt][dt][1], O[qt][dt][2], O[qt][dt][3]);
        if (kq == 0) S.m_w[wave][r] = m[qt], S.l_w[wave][r] = l[qt];
    }
    __syncthreads();
    // The work item's (m, l) per row from its waves' (a thread per row; the
    // waves' weights 2^(m_w - M) overwrite their m), then its O.
    // Row r is local row r % MQ_WR of the MQ_KG waves of set r / MQ_WR.
    if (tid < MQ_ROWS) {
        const int w0 = (tid / MQ_WR) * MQ_KG, lr = tid % MQ_WR;
        float M = S.m_w[w0][lr];
#pragma unroll
        for (int w = 1; w < MQ_KG; w++) M = fmaxf(M, S.m_w[w0 + w][lr]);
        float L = 0.f;
#pragma unroll
        for (int w = 0; w < MQ_KG; w++) {
            const float wt = S.m_w[w0 + w][lr] == -INFINITY ? 0.f : exp2f(S.m_w[w0 + w][lr] - M);
            L += wt * S.l_w[w0 + w][lr];
            S.m_w[w0 + w][lr] = wt;
        }
        S.l_w[w0][lr] = M, S.l_w[w0 + 1][lr] = L;
    }
    __syncthreads();
    auto item = [&](int r, int d, float &M, float &L) {
        const int w0 = (r / MQ_WR) * MQ_KG, lr = r % MQ_WR;
        float Ov = 0.f;
#pragma unroll
        for (int w = 0; w < MQ_KG; w++) Ov += S.m_w[w0 + w][lr] * S.o_w[w0 + w][lr][4 + d];
        M = S.l_w[w0][lr], L = S.l_w[w0 + 1][lr];
        return Ov;
    };
    // The partial, merged by k_attn_mq_merge (the next launch on the stream;
    // also with one used split).
    float *rec = a.part + ((int64_t)split * a.HKV + kvh) * R * MQ_REC;
    for (int j = tid; j < R * MQ_HD; j += MQ_NT) {
        const int r = j / MQ_HD, d = j % MQ_HD;
        float M, L;
        rec[r * MQ_REC + 4 + d] = item(r, d, M, L);
        if (d == 0) rec[r * MQ_REC] = M, rec[r * MQ_REC + 1] = L;
    }
}

// 3. The merge of the used splits' partials for row r of KV head kvh (one
// workgroup, a thread per dimension): out = sum_s 2^(m_s - M) O_s /
// sum_s 2^(m_s - M) l_s in split order (attn_merge.comp:18-47), every
// split's value requested before any is added; with act_out, the head's 128
// values also as 8 runs of the token's activation records (quant_run_m, as
// k_act_quant_m writes them).
__device__ inline void attn_mq_merge(const AttnArgs &a, int G, int B, int n_split, int r, int kvh) {
    __shared__ float wts[ATTN_MAX_SPLIT], wl[ATTN_MAX_SPLIT], ov[MQ_HD];
    const int d = threadIdx.x, R = B * G;
    const int nk = a.n_keys[0] + B;
    int chunk = (nk + n_split - 1) / n_split;
    chunk = (chunk + MQ_STEP - 1) / MQ_STEP * MQ_STEP;
    const int used = (nk + chunk - 1) / chunk;
    const int64_t sstride = (int64_t)a.HKV * R * MQ_REC;
    const float *p = a.part + ((int64_t)kvh * R + r) * MQ_REC;
    constexpr int SB = 32;  // splits whose values are requested with the weights
    float o[SB];
#pragma unroll
    for (int j = 0; j < SB; j++) o[j] = p[min(j, used - 1) * sstride + 4 + d];
    if (d < 64) {
        const int sl = min(d, used - 1);
        const float ms = d < used ? p[sl * sstride] : -INFINITY, ls = p[sl * sstride + 1];
        const float M = wave_max_dpp(ms);
        const float w = ms == -INFINITY ? 0.f : exp2f(ms - M);
        wts[d] = w, wl[d] = w * ls;
    }
    __syncthreads();
    float den = 0.f, num = 0.f;
    for (int s2 = 0; s2 < used; s2++) den += wl[s2];
    for (int s0 = 0; s0 < used; s0 += SB) {
        if (s0) {
#pragma unroll
            for (int j = 0; j < SB; j++) o[j] = p[min(s0 + j, used - 1) * sstride + 4 + d];
        }
#pragma unroll
        for (int j = 0; j < SB; j++)
            if (s0 + j < used) num += wts[s0 + j] * o[j];
    }
    const float res = den > 0.f ? num / den : 0.f;
    const int b = r / G, h = kvh * G + r % G;
    a.out[(int64_t)b * a.H * MQ_HD + (int64_t)h * MQ_HD + d] = res;
    if (!a.act_out) return;
    ov[d] = res;
    __syncthreads();
    if (d < MQ_HD / 16) {  // runs 8 h .. 8 h + 7, pairs in adjacent lanes
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = ov[16 * d + i];
        quant_run_m(v, (MQ_HD / 16) * h + d, a.act_out + (int64_t)b * a.act_stride);
    }
}

}  // namespace ts5hip
