// Split-K decode attention of one query per (key slice, KV head, query) work
// item on the matrix cores, for a q8 or f16 cache at head dimension 128: the work
// items of k_attn (attn_core.h; the same spans, preparation, partials and
// merge, engine/src/cpu_backend.cpp:224-248 per query, attn_merge.comp:18-47)
// with the key loop of the multi-query kernel (attn_mq.h) on one 16-row tile
// whose first G rows are the query's heads. Used where k_attn took one query
// per cache: caches past the LDS kernel's reach and batches of queries on
// caches of their own (kv_per_batch). Per-query k_attn spends about 650 VALU
// instructions a lane per 16 keys (the q.k and p.v multiply-adds, the int8
// conversions), which bounds it near 3.7 TB/s at 16 queries x 32768 keys.
//
// 8 waves; each takes 16 keys of every 128-key step of the slice:
//   S^T (16 keys x 16 rows) = K . Q^T on v_mfma_f32_16x16x32_f16, each row as
//   fp16 hi + lo planes of q * scale * 2^-e (e per row); q8: per 32-value
//   scale group, K as exact fp16 integers, then S += ks * R; f16: K as it is
//   stored, one sum over the 128 dims;
//   online softmax per row (the rows are the lanes' columns);
//   O^T (128 dims x 16 rows) += V^T . (P o vs)^T on v_mfma_f32_16x16x16_f16,
//   V (q8: exact integers; f16: as stored) transposed through the wave's own
//   LDS, 128 P o vs (vs = 1 for f16) as fp16 hi + lo (the D layout of S^T is
//   the B layout: P stays in registers; the factor 128 keeps its lo plane
//   out of the f16 subnormals and leaves O at the end).
// The waves' (m, l, O) then go through attn_item_out like k_attn's.
#pragma once
#include <type_traits>

#include "attn_mq.h"

namespace ts5hip {

constexpr int M1_NW = 8, M1_NT = 64 * M1_NW;  // waves and threads of a work item
constexpr int M1_STEP = 16 * M1_NW;            // keys of a work item's step

template <int G>
struct M1Lds {
    float q_s[G][MQ_HD];
    float m_s[G], l_s[G], red[G];
    // The new keys before rounding live until the preparation's last
    // barrier; the waves' results are written after the key loop.
    union {
        float kv_s[ATTN_MAX_NEW][2][MQ_HD];
        struct {
            __align__(16) float o_w[M1_NW][G][MQ_HD];
            float m_w[M1_NW][G], l_w[M1_NW][G];
        };
    };
    union {
        struct {
            __align__(16) int8_t new8[ATTN_MAX_NEW][2][MQ_HD];
            uint16_t new_sc[ATTN_MAX_NEW][2][MQ_HD / 32];
        };
        __align__(16) uint16_t new16[ATTN_MAX_NEW][2][MQ_HD];
    };
    __align__(16) uint32_t vt[M1_NW][MQ_HD * MQ_VT];  // each wave's 16 keys' V^T, [d][key quad] as f16
    __align__(16) float wts[G][ATTN_MAX_SPLIT];
    int last;
};

template <int G, bool F16>
__device__ inline void attn_m1(const AttnArgs &a, int split, int kvh, int b, int n_split, M1Lds<G> &S) {
    static_assert(G >= 1 && G <= 16, "the query heads fit one 16-row tile");
    constexpr int HD = MQ_HD;
    constexpr int VB = F16 ? 2 : 1;  // bytes per cached value
    constexpr float LOG2E = 1.4426950408889634f;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int rl = lane & 15, kq = lane >> 4;
    const bool row_ok = rl < G;  // the lane's column is one of the query's heads
    const AttnSpan sp = attn_span<16>(a, split, kvh, b, n_split);
    if (split >= sp.used) return;  // an empty split: not counted, not merged
    const int nkeys = max(sp.p1 - sp.p0, 0);
    // The slice's K and V (and scales) as bounded buffers from key p0: past
    // p1 they read zeros and touch no memory.
    const int64_t base = sp.head_base + sp.p0;
    const __amdgpu_buffer_rsrc_t rk = slice_rsrc(a.kv.k + base * HD * VB, (uint32_t)nkeys * HD * VB);
    const __amdgpu_buffer_rsrc_t rv = slice_rsrc(a.kv.v + base * HD * VB, (uint32_t)nkeys * HD * VB);
    __amdgpu_buffer_rsrc_t rks = rk, rvs = rv;  // q8: the scales (an f16 cache has none)
    if constexpr (!F16) {
        rks = slice_rsrc(a.kv.ks + base * 4, (uint32_t)nkeys * 8);
        rvs = slice_rsrc(a.kv.vs + base * 4, (uint32_t)nkeys * 8);
    }
    // A step's loads for this wave's 16 keys kl .. kl + 15 (relative to p0):
    // K: key kl + rl, dims 32 c + 8 kq .. + 7 (the A operand of group c);
    // V: keys kl + 4 kq + i, dims 8 rl .. 8 rl + 7 (the lane's share of the
    // transpose); q8: the K and V scales of keys kl + 4 kq + i (the lane's S
    // and P entries), all 4 groups.
    using Piece = std::conditional_t<F16, u32x4, u32x2>;  // 8 values
    struct Step {
        Piece k[4], v[4];
        u32x4 ks[F16 ? 1 : 2], vs[F16 ? 1 : 2];
    };
    auto piece = [&](__amdgpu_buffer_rsrc_t r, uint32_t e) -> Piece {  // values e .. e + 7
        if constexpr (F16) return __builtin_amdgcn_raw_buffer_load_b128(r, e * 2, 0, 0);
        else return __builtin_amdgcn_raw_buffer_load_b64(r, e, 0, 0);
    };
    auto load = [&](Step &w, int st) {
        const uint32_t kl = (uint32_t)(st * M1_STEP + wave * 16);
#pragma unroll
        for (int c = 0; c < 4; c++) w.k[c] = piece(rk, (kl + rl) * HD + 32 * c + 8 * kq);
#pragma unroll
        for (int i = 0; i < 4; i++) w.v[i] = piece(rv, (kl + 4 * kq + i) * HD + 8 * rl);
        if constexpr (!F16) {
#pragma unroll
            for (int h = 0; h < 2; h++) {
                w.ks[h] = __builtin_amdgcn_raw_buffer_load_b128(rks, (kl + 4 * kq) * 8 + 16 * h, 0, 0);
                w.vs[h] = __builtin_amdgcn_raw_buffer_load_b128(rvs, (kl + 4 * kq) * 8 + 16 * h, 0, 0);
            }
        }
    };
    // The 8 values of a piece as the MFMA operand.
    auto values = [&](const Piece &p) -> mq_h8 {
        if constexpr (F16) return __builtin_bit_cast(mq_h8, p);
        else return mq_i8x8(p[0], p[1]);
    };
    // The query's inputs are requested first, then the first three steps'
    // K and V (loads complete in order: the preparation then waits for its
    // own inputs only), unless the slice holds the new key: the preparation
    // stores it at its cache slot, and the slice is read after those stores
    // are complete.
    AttnPre<HD, G, M1_NT> pre;
    attn_preload<HD, G, M1_NT>(a, kvh, b, sp, pre);
    Step A, Bs, Cs;
    if (!sp.has_new) load(A, 0), load(Bs, 1), load(Cs, 2);
    attn_prepare<HD, G, M1_NT, F16>(a, kvh, b, sp, S, &pre);
    if (sp.has_new) {
        wait_stores();
        __syncthreads();
        load(A, 0), load(Bs, 1), load(Cs, 2);
    }
    // The lane's row (its MFMA column) as B operands: dims 32 c + 8 kq .. + 7
    // of q * scale * 2^-e, hi and lo; rows past G are zero and take no key.
    mq_h8 qh[4], ql[4];
    float p2e;
    {
        const int r = row_ok ? rl : 0;
        float v[4][8], amax = 0.f;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float4 x0 = *(const float4 *)&S.q_s[r][32 * c + 8 * kq];
            const float4 x1 = *(const float4 *)&S.q_s[r][32 * c + 8 * kq + 4];
            const float f[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) v[c][j] = row_ok ? f[j] * a.scale : 0.f, amax = fmaxf(amax, fabsf(v[c][j]));
        }
        amax = max_xor32(max_xor16(amax));
        const int e = amax > 0.f ? max(ilogbf(amax) - 13, -100) : 0;
        const float sc = ldexpf(1.0f, -e);
        p2e = ldexpf(1.0f, e);
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float f = v[c][j] * sc;  // exact: sc is a power of 2
                qh[c][j] = (_Float16)f;
                ql[c][j] = (_Float16)(f - (float)qh[c][j]);
            }
    }

    mq_f4 O[8];
    float m = -INFINITY, l = 0.f;
#pragma unroll
    for (int dt = 0; dt < 8; dt++) O[dt] = mq_f4{0.f, 0.f, 0.f, 0.f};
    uint32_t *vt = S.vt[wave];
    auto step = [&](const Step &w, int st) {
        const int kl = st * M1_STEP + wave * 16;
        // q8 scales: halfword 4 i + c of the pair of u32x4 is key kl + 4 kq + i, group c.
        float ksf[4][4], vsf[4][4];
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int hw = 4 * i + c;
                ksf[i][c] = F16 ? 1.f : h2f((w.ks[hw >> 3][(hw >> 1) & 3] >> (16 * (hw & 1))) & 0xffff);
                vsf[i][c] = F16 ? 1.f : h2f((w.vs[hw >> 3][(hw >> 1) & 3] >> (16 * (hw & 1))) & 0xffff);
            }
        // S^T: D[key 4 kq + i][row rl].
        float s[4];
        if constexpr (F16) {  // one sum over the 128 dims
            mq_f4 R = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const mq_h8 ka = values(w.k[c]);
                R = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[c], R, 0, 0, 0);
                R = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[c], R, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; i++) s[i] = R[i];
        } else {  // a sum per scale group, scaled
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const mq_h8 ka = values(w.k[c]);
                mq_f4 R = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[c], mq_f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                R = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[c], R, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++) s[i] = c == 0 ? ksf[i][c] * R[i] : fmaf(ksf[i][c], R[i], s[i]);
            }
        }
        // V^T of the wave's 16 keys into its LDS: dim d = 8 rl + j, key quad
        // kq (keys 4 kq + i) as 4 f16 at dword MQ_VT d + 2 kq, each value the
        // exact integer v8 or the f16 value (P carries the scale times 128, O
        // the factor 128 until the end).
        {
            mq_h8 hv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) hv[i] = values(w.v[i]);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const mq_h4 col = {hv[0][j], hv[1][j], hv[2][j], hv[3][j]};
                *(mq_h4 *)&vt[(8 * rl + j) * MQ_VT + 2 * kq] = col;
            }
        }
        // Online softmax of the lane's row (natural-log domain, as k_attn's
        // partials), then the B operands (P o vs of group g) as hi + lo.
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int key = kl + 4 * kq + i;
            const float sv = row_ok && key < nkeys ? s[i] * p2e : -INFINITY;
            s[i] = sv;
            mx = fmaxf(mx, sv);
        }
        mx = max_xor32(max_xor16(mx));
        const float mn = fmaxf(m, mx);
        const float alpha = mn == -INFINITY ? 1.0f : __builtin_amdgcn_exp2f((m - mn) * LOG2E);
        float p[4], sum = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            p[i] = mn == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((s[i] - mn) * LOG2E);
            sum += p[i];
            p[i] *= 128.f;  // exact; keeps the lo plane of p * vs out of the f16 subnormals
        }
        sum = add_xor32(add_xor16(sum));
        m = mn, l = l * alpha + sum;
        if (alpha != 1.0f) {
#pragma unroll
            for (int dt = 0; dt < 8; dt++) O[dt] *= alpha;
        }
        // x = 128 p * vs rounded to fp32 before its split (the empty asm
        // keeps a contracted product out of the conversions), so that hi + lo
        // is x.
        mq_h4 ph[4], pl[4];
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float x = p[i] * vsf[i][g];
                asm volatile("" : "+v"(x));
                ph[g][i] = (_Float16)x;
                pl[g][i] = (_Float16)(x - (float)ph[g][i]);
            }
        // O^T += V^T (P o vs)^T: A = V^T rows 16 dt + rl, keys 4 kq .. + 3
        // (the wave's own LDS writes above are in: one wave, in order).
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
#pragma unroll
        for (int dt = 0; dt < 8; dt++) {
            const mq_h4 va = *(const mq_h4 *)&vt[(16 * dt + rl) * MQ_VT + 2 * kq];
            O[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, ph[dt >> 1], O[dt], 0, 0, 0);
            O[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, pl[dt >> 1], O[dt], 0, 0, 0);
        }
        // The next step's V^T writes must not pass these reads: in order.
    };
    // Three register sets in turn; each is refilled with the step three on
    // as soon as it is used (past the slice: zeros, no memory access). The
    // loop's iteration has no exit but its end, so that the compiler's wait
    // for a step's loads leaves the two later steps' in flight (an exit
    // between the steps made it wait for all of them); the last one or two
    // steps follow it.
    const int nsteps = (nkeys + M1_STEP - 1) / M1_STEP;
    int st = 0;
    for (; st + 3 <= nsteps; st += 3) {
        step(A, st);
        load(A, st + 3);
        step(Bs, st + 1);
        load(Bs, st + 4);
        step(Cs, st + 2);
        load(Cs, st + 5);
    }
    if (st < nsteps) step(A, st);
    if (st + 1 < nsteps) step(Bs, st + 1);
    // The wave's rows: O^T[d = 16 dt + 4 kq + i][row rl], and (m, l). The
    // preparation's reads of kv_s, which o_w overlays, ended at its last
    // barrier.
    if (row_ok) {
        constexpr float k2m7 = 0.0078125f;  // the factor 128 out (exact)
#pragma unroll
        for (int dt = 0; dt < 8; dt++)
            *(float4 *)&S.o_w[wave][rl][16 * dt + 4 * kq] =
                make_float4(O[dt][0] * k2m7, O[dt][1] * k2m7, O[dt][2] * k2m7, O[dt][3] * k2m7);
        if (kq == 0) S.m_w[wave][rl] = m, S.l_w[wave][rl] = l;
    }
    __syncthreads();
    attn_item_out<HD, G, M1_NT>(a, sp, split, kvh, b, n_split, S);
}

}  // namespace ts5hip
