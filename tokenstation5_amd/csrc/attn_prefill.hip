// Prompt attention over the q8 (or f16) KV cache on the matrix cores: causal
// flash attention for a batch of consecutive queries (positions p0 .. p0 +
// nq - 1) against keys 0 .. p0 + t (the reference's attn_pf path,
// engine/shaders/attn_pf.glsl, attn_pf_q8.comp and attn_pf128.comp, with its
// policy in engine/src/vk_backend.cpp:954-975; the CPU restatement
// engine/src/cpu_backend.cpp:224-248). Head dimension 64 or 128.
//
// Workgroup: one KV head, QB = floor(128 / G) queries (G QB of its 128 query
// rows: query t, group head j at row G t + j), one split of the keys
// (split_keys, a multiple of 64). Four waves, 32 query rows (two 16-row
// tiles) each. Keys go in blocks of 64:
//  * DMA brings the block's raw q8 keys and values (and their f16 scales) into
//    LDS while the previous block is computed; all 256 threads then convert
//    them: K to exact fp16 integers (k8), V to exact fp16 hi + lo planes of
//    v8 * vs, transposed ([d][key]) for the value product.
//  * S^T (keys x rows) = K . Q^T on v_mfma_f32_16x16x32_f16, per 32-value
//    group of the head dimension (one q8 scale group): the query rows are
//    fp16 hi + lo planes of q * scale * log2(e) * 2^-e (e per row keeps them in
//    range), two MFMAs into one fp32 accumulator, then S += ks * R per group.
//  * online softmax per row in the log2 domain (causal mask, running max m and
//    sum l; the rows are the lanes' columns, so only 4-lane exchanges).
//  * O^T (d x rows) += V^T . P^T on v_mfma_f32_16x16x16_f16, whose B operand
//    layout is exactly the D layout of the S^T tiles: P stays in registers as
//    fp16 hi + lo; Vh Ph + Vl Ph + Vh Pl.
// Several key splits write (m, l, O) partials that a second kernel merges in
// split order; one split writes O / l directly.
//
// An f16 cache (the reference's default KV type) takes the same kernel with
// K and V as stored: DMA brings K straight into the fp16 tile layout (two
// buffers, the next block's while this one is computed), V's raw block is
// transposed into V^T, S needs no scale and the value product no lo plane of
// V (Vh Ph + Vh Pl).
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace ts5hip {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

struct PfArgs {
    const float *q;  // query rows [nq][q_stride], head hh at hh * HD
    int64_t q_stride;
    KvLayer kv;
    int n_ctx, H, HKV, p0, nq, n_split, split_keys;
    float scale;
    float *part;  // [nq][H][n_split][HD + 4]: m, l, -, -, O[HD]
    float *out;   // [nq][H * HD]
};

constexpr int PF_KB = 64;     // keys per block
constexpr int PF_ROWS = 128;  // query rows per workgroup
// The k16 tiles' swizzle: unit u of key k sits at u ^ (k & pf_ksw(HD)), a
// permutation of the key's HD / 8 units.
__host__ __device__ constexpr int pf_ksw(int hd) { return hd / 8 - 1 < 15 ? hd / 8 - 1 : 15; }
constexpr float PF_LOG2E = 1.4426950408889634f;

template <int HD, bool F16>
struct PfLds;

template <int HD>
struct PfLds<HD, false> {
    int8_t k8[PF_KB][HD];          // raw blocks (DMA)
    int8_t v8[PF_KB][HD];
    uint16_t ks[PF_KB][HD / 32];
    uint16_t vs[PF_KB][HD / 32];
    uint4 k16[PF_KB][HD / 8];      // k8 as fp16, unit u of key k at u ^ (k & pf_ksw(HD))
    float ksf[HD / 32][PF_KB];     // K scales, [group][key]
    uint2 vh[HD][PF_KB / 4];       // V^T hi, key quad q of row d at q ^ (d & 15)
    uint2 vl[HD][PF_KB / 4];       // V^T lo
};

template <int HD>
struct PfLds<HD, true> {
    uint4 k16[2][PF_KB][HD / 8];  // K as stored (DMA), unit u of key k at u ^ (k & pf_ksw(HD)); two blocks in turn
    uint16_t v16[PF_KB][HD];      // raw V block (DMA)
    uint2 vh[HD][PF_KB / 4];      // V^T, key quad q of row d at q ^ (d & 15)
};

// Raw block at key kb (keys past n_ctx read the last slot; they are masked).
template <int HD>
__device__ inline void pf_issue(const PfArgs &a, PfLds<HD, false> &L, int64_t slot0, int kb, int wave, int lane, int) {
    constexpr int PIECES = PF_KB * HD / 16;  // 16-byte pieces per plane
    constexpr int PER_WAVE = PIECES / 64 / 4;
#pragma unroll
    for (int i = 0; i < PER_WAVE; i++) {
        const int j = wave * PER_WAVE + i, u = 64 * j + lane, key = u / (HD / 16), piece = u % (HD / 16);
        const int64_t slot = slot0 + min(kb + key, a.n_ctx - 1);
        dma16(a.kv.k + slot * HD + 16 * piece, lds_addr(&L.k8[0][0]) + 1024 * j);
        dma16(a.kv.v + slot * HD + 16 * piece, lds_addr(&L.v8[0][0]) + 1024 * j);
    }
    {  // scales: 64 keys x HD / 32 f16 = DW dwords a plane, WPP waves a plane (dwords 64 (w % WPP) + lane)
        constexpr int DW = PF_KB * (HD / 32) / 2, WPP = DW / 64;
        static_assert(DW % 64 == 0 && 2 * WPP <= 4, "whole dword DMAs, both planes in four waves");
        if (WPP == 2 || wave < 2 * WPP) {  // (four waves: every wave)
            const int plane = wave / WPP, w = 64 * (wave % WPP) + lane, key = w / (HD / 64);
            const uint16_t *base = plane ? a.kv.vs : a.kv.ks;
            const uint16_t *src = base + (slot0 + min(kb + key, a.n_ctx - 1)) * (HD / 32) + 2 * (w % (HD / 64));
            dma4(src, lds_addr(plane ? &L.vs[0][0] : &L.ks[0][0]) + 256 * (wave % WPP));
        }
    }
}

// An f16 block at key kb: K into k16[buf] (LDS piece p = 64 j + lane is
// unit p % (HD / 8) ^ (key & pf_ksw(HD)) of key p / (HD / 8)), V raw into v16.
template <int HD>
__device__ inline void pf_issue(const PfArgs &a, PfLds<HD, true> &L, int64_t slot0, int kb, int wave, int lane,
                                int buf) {
    constexpr int UNITS = HD / 8;                     // 16-byte units of a key
    constexpr int PER_WAVE = PF_KB * UNITS / 64 / 4;  // 1024-byte requests a wave, per plane
    const int8_t *kbase = (const int8_t *)a.kv.k, *vbase = (const int8_t *)a.kv.v;
#pragma unroll
    for (int i = 0; i < PER_WAVE; i++) {
        const int j = wave * PER_WAVE + i, p = 64 * j + lane, key = p / UNITS, pos = p % UNITS;
        const int64_t slot = slot0 + min(kb + key, a.n_ctx - 1);
        dma16(kbase + slot * HD * 2 + 16 * (pos ^ (key & pf_ksw(HD))), lds_addr(&L.k16[buf][0][0]) + 1024 * j);
        dma16(vbase + slot * HD * 2 + 16 * pos, lds_addr(&L.v16[0][0]) + 1024 * j);
    }
}

// Raw V -> V^T (keys at or past kend: V = 0); K is already in place.
template <int HD>
__device__ inline void pf_convert(PfLds<HD, true> &L, int kb, int kend) {
    constexpr int DQ = HD / 4;  // d quads; thread = (4 consecutive d, 8 consecutive keys)
    for (int w = threadIdx.x; w < DQ * (PF_KB / 8); w += 256) {
        const int dq = w % DQ, k0 = 8 * (w / DQ), d0 = 4 * dq;
        uint32_t hw[4][4];  // [d][key pair]
#pragma unroll
        for (int kk = 0; kk < 8; kk += 2) {
            uint2 r[2];
#pragma unroll
            for (int e = 0; e < 2; e++) {
                const int key = k0 + kk + e;
                r[e] = kb + key < kend ? *(const uint2 *)&L.v16[key][d0] : make_uint2(0u, 0u);
            }
            hw[0][kk / 2] = (r[0].x & 0xffffu) | (r[1].x << 16);
            hw[1][kk / 2] = (r[0].x >> 16) | (r[1].x & 0xffff0000u);
            hw[2][kk / 2] = (r[0].y & 0xffffu) | (r[1].y << 16);
            hw[3][kk / 2] = (r[0].y >> 16) | (r[1].y & 0xffff0000u);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int d = d0 + j, q0 = k0 / 4;
            L.vh[d][q0 ^ (d & 15)] = make_uint2(hw[j][0], hw[j][1]);
            L.vh[d][(q0 + 1) ^ (d & 15)] = make_uint2(hw[j][2], hw[j][3]);
        }
    }
}

// Raw -> K16, ksf, V^T hi/lo (keys at or past kend: V = 0).
template <int HD>
__device__ inline void pf_convert(PfLds<HD, false> &L, int kb, int kend) {
    const int t = threadIdx.x;
    {  // K: thread t converts 8 * HD / 256 ... one key quarter of 32 values
        constexpr int PER_KEY = HD / 32;  // threads per key
        for (int w = t; w < PF_KB * PER_KEY; w += 256) {
            const int key = w / PER_KEY, part = w % PER_KEY;  // 32 values: units 4 part .. 4 part + 3
            const uint4 r0 = *(const uint4 *)&L.k8[key][32 * part], r1 = *(const uint4 *)&L.k8[key][32 * part + 16];
            const uint32_t words[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
            uint32_t h[16];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                const uint32_t v = words[k] ^ 0x80808080u;  // b + 128, then 0x64xx = 1024 + b + 128
                const v2h k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
                h[2 * k] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, v, 0x04010400u)) - k1152);
                h[2 * k + 1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, v, 0x04030402u)) - k1152);
            }
#pragma unroll
            for (int k = 0; k < 4; k++)
                L.k16[key][(4 * part + k) ^ (key & pf_ksw(HD))] =
                    make_uint4(h[4 * k], h[4 * k + 1], h[4 * k + 2], h[4 * k + 3]);
        }
    }
    if (t < PF_KB * (HD / 32)) {
        const int key = t / (HD / 32), grp = t % (HD / 32);
        L.ksf[grp][key] = h2f(L.ks[key][grp]);
    }
    {  // V^T: thread = (4 consecutive d, 8 consecutive keys)
        constexpr int DQ = HD / 4;  // d quads
        for (int w = t; w < DQ * (PF_KB / 8); w += 256) {
            const int dq = w % DQ, k0 = 8 * (w / DQ), d0 = 4 * dq;
            uint32_t hw[4][4], lw[4][4];  // [d][key pair]
#pragma unroll
            for (int kk = 0; kk < 8; kk += 2) {
                float f[2][4];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const int key = k0 + kk + e;
                    const uint32_t raw = *(const uint32_t *)&L.v8[key][d0];
                    const float s = kb + key < kend ? h2f(L.vs[key][d0 / 32]) : 0.f;
#pragma unroll
                    for (int j = 0; j < 4; j++) f[e][j] = (float)(int8_t)(raw >> (8 * j)) * s;
                }
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const _Float16 h0 = (_Float16)f[0][j], h1 = (_Float16)f[1][j];
                    const _Float16 l0 = (_Float16)(f[0][j] - (float)h0), l1 = (_Float16)(f[1][j] - (float)h1);
                    hw[j][kk / 2] = __builtin_bit_cast(uint16_t, h0) | (uint32_t)__builtin_bit_cast(uint16_t, h1) << 16;
                    lw[j][kk / 2] = __builtin_bit_cast(uint16_t, l0) | (uint32_t)__builtin_bit_cast(uint16_t, l1) << 16;
                }
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int d = d0 + j, q0 = k0 / 4;
                L.vh[d][q0 ^ (d & 15)] = make_uint2(hw[j][0], hw[j][1]);
                L.vh[d][(q0 + 1) ^ (d & 15)] = make_uint2(hw[j][2], hw[j][3]);
                L.vl[d][q0 ^ (d & 15)] = make_uint2(lw[j][0], lw[j][1]);
                L.vl[d][(q0 + 1) ^ (d & 15)] = make_uint2(lw[j][2], lw[j][3]);
            }
        }
    }
}

// GT: the query group as a constant, or 0 to take it from the arguments;
// rows past G QB (G not a power of two) are idle.
template <int HD, int GT, bool F16>
__global__ __launch_bounds__(256, 2) void k_attn_pf(PfArgs a) {
    constexpr int NC = HD / 32, NDT = HD / 16, KSW = pf_ksw(HD);
    const int G = GT ? GT : a.H / a.HKV, QB = PF_ROWS / G;
    constexpr bool FULL = GT && PF_ROWS % GT == 0;  // every row a query's
    __shared__ PfLds<HD, F16> L;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, kq = lane >> 4, rl = lane & 15;
    const int h = blockIdx.y, t0 = blockIdx.x * QB, sp = blockIdx.z;
    const int t_last = min(a.nq, t0 + QB) - 1;
    const int kbeg = sp * a.split_keys;
    const int kend = min(kbeg + a.split_keys, a.p0 + t_last + 1);  // keys past every row's limit are not read
    if (kbeg >= kend) return;  // the merge reads no partial of this split
    const int64_t slot0 = (int64_t)h * a.n_ctx;

    // The lane's query rows (its MFMA columns): row 32 wave + 16 qt + rl.
    int pos[2];  // the rows' positions (the causal limit); their query and head again at the end
    float p2e[2];
    v8h qh[2][NC], ql[2][NC];
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const int r = 32 * wave + 16 * qt + rl;
        const int tq = t0 + r / G, hh = h * G + r % G;
        pos[qt] = a.p0 + tq;
        const float *qr = a.q + (int64_t)min(tq, a.nq - 1) * a.q_stride + (int64_t)hh * HD + 8 * kq;
        float v[NC][8], amax = 0.f;
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const float4 x0 = *(const float4 *)(qr + 32 * c), x1 = *(const float4 *)(qr + 32 * c + 4);
            const float f[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int j = 0; j < 8; j++) v[c][j] = f[j] * (a.scale * PF_LOG2E), amax = fmaxf(amax, fabsf(v[c][j]));
        }
        amax = max_xor32(max_xor16(amax));
        const int e = amax > 0.f ? max(ilogbf(amax) - 13, -100) : 0;
        const float sc = ldexpf(1.0f, -e);
        p2e[qt] = ldexpf(1.0f, e);
#pragma unroll
        for (int c = 0; c < NC; c++)
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const float f = v[c][j] * sc;
                qh[qt][c][j] = (_Float16)f;
                ql[qt][c][j] = (_Float16)(f - (float)qh[qt][c][j]);
            }
    }

    v4f O[2][NDT];
    float m[2], l[2];
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        m[qt] = -INFINITY, l[qt] = 0.f;
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) O[qt][dt] = v4f{0.f, 0.f, 0.f, 0.f};
    }

    pf_issue<HD>(a, L, slot0, kbeg, wave, lane, 0);
    for (int kb = kbeg, nb = 0; kb < kend; kb += PF_KB, nb++) {
        wait_vm_n<0>();
        __syncthreads();  // the raw block is in; every wave is done with the last block's K16 / V^T
        pf_convert<HD>(L, kb, kend);
        __syncthreads();  // K16 / V^T ready; the raw buffers are free
        if (kb + PF_KB < kend) pf_issue<HD>(a, L, slot0, kb + PF_KB, wave, lane, (nb + 1) & 1);

        // S^T tiles: keys kb + 16 kt + 4 kq + i, row columns.
        float S[4][2][4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            const int key = 16 * kt + rl;
            if constexpr (F16) {  // K as stored: one sum over the head dimension
                v4f R[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    const v8h A = __builtin_bit_cast(v8h, L.k16[nb & 1][key][(4 * c + kq) ^ (key & KSW)]);
#pragma unroll
                    for (int qt = 0; qt < 2; qt++) {
                        R[qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, qh[qt][c], R[qt], 0, 0, 0);
                        R[qt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, ql[qt][c], R[qt], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int qt = 0; qt < 2; qt++)
#pragma unroll
                    for (int i = 0; i < 4; i++) S[kt][qt][i] = R[qt][i];
            } else {
#pragma unroll
                for (int c = 0; c < NC; c++) {
                    const v8h A = __builtin_bit_cast(v8h, L.k16[key][(4 * c + kq) ^ (key & KSW)]);
                    const float4 ks4 = *(const float4 *)&L.ksf[c][16 * kt + 4 * kq];
                    const float ksv[4] = {ks4.x, ks4.y, ks4.z, ks4.w};
#pragma unroll
                    for (int qt = 0; qt < 2; qt++) {
                        v4f R = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, qh[qt][c], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        R = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, ql[qt][c], R, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            S[kt][qt][i] = c == 0 ? ksv[i] * R[i] : fmaf(ksv[i], R[i], S[kt][qt][i]);
                    }
                }
            }
        }
        // Online softmax per row (log2 domain).
        v4h ph[4][2], pl[4][2];
#pragma unroll
        for (int qt = 0; qt < 2; qt++) {
            float mx = -INFINITY;
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int key = kb + 16 * kt + 4 * kq + i;
                    const float s = key <= pos[qt] && key < kend ? S[kt][qt][i] * p2e[qt] : -INFINITY;
                    S[kt][qt][i] = s;
                    mx = fmaxf(mx, s);
                }
            mx = max_xor32(max_xor16(mx));
            const float mn = fmaxf(m[qt], mx);
            const float alpha = mn == -INFINITY ? 1.0f : exp2f(m[qt] - mn);
            float sum = 0.f;
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float p = mn == -INFINITY ? 0.f : exp2f(S[kt][qt][i] - mn);
                    sum += p;
                    ph[kt][qt][i] = (_Float16)p;
                    pl[kt][qt][i] = (_Float16)(p - (float)ph[kt][qt][i]);
                }
            sum = add_xor32(add_xor16(sum));
            m[qt] = mn, l[qt] = l[qt] * alpha + sum;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++) O[qt][dt] *= alpha;
        }
        // O^T += V^T P^T.
#pragma unroll
        for (int dt = 0; dt < NDT; dt++) {
            const int d = 16 * dt + rl;
#pragma unroll
            for (int kt = 0; kt < 4; kt++) {
                const int quad = 4 * kt + kq;
                const v4h vh = __builtin_bit_cast(v4h, L.vh[d][quad ^ (d & 15)]);
#pragma unroll
                for (int qt = 0; qt < 2; qt++) {
                    O[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vh, ph[kt][qt], O[qt][dt], 0, 0, 0);
                    if constexpr (!F16) {
                        const v4h vl = __builtin_bit_cast(v4h, L.vl[d][quad ^ (d & 15)]);
                        O[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vl, ph[kt][qt], O[qt][dt], 0, 0, 0);
                    }
                    O[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vh, pl[kt][qt], O[qt][dt], 0, 0, 0);
                }
            }
        }
    }

    // Rows of this lane's columns: O^T[d = 16 dt + 4 kq + i][row].
#pragma unroll
    for (int qt = 0; qt < 2; qt++) {
        const int r = 32 * wave + 16 * qt + rl, tq = t0 + r / G, hh = h * G + r % G;
        if (tq >= a.nq || (!FULL && r >= G * QB)) continue;
        if (a.n_split == 1) {
            const float inv = 1.0f / l[qt];
            float *o = a.out + (int64_t)tq * a.H * HD + (int64_t)hh * HD;
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                *(float4 *)(o + 16 * dt + 4 * kq) =
                    make_float4(O[qt][dt][0] * inv, O[qt][dt][1] * inv, O[qt][dt][2] * inv, O[qt][dt][3] * inv);
        } else {
            float *p = a.part + (((int64_t)tq * a.H + hh) * a.n_split + sp) * (HD + 4);
            if (kq == 0) p[0] = m[qt], p[1] = l[qt];
#pragma unroll
            for (int dt = 0; dt < NDT; dt++)
                *(float4 *)(p + 4 + 16 * dt + 4 * kq) = make_float4(O[qt][dt][0], O[qt][dt][1], O[qt][dt][2], O[qt][dt][3]);
        }
    }
}

// out[t][hh] = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s over the splits
// that hold keys of row t (s * split_keys <= p0 + t), in split order.
constexpr int PF_MAX_SPLIT = 64;  // partials a row can merge (k_attn_pf makes at most 16)

template <int HD>
__global__ __launch_bounds__(HD) void k_attn_pf_merge(PfArgs a) {
    // The splits' weights 2^(m_s - M) and w_s l_s: wave 0, a lane per split;
    // their sum in split order; then each thread's d over every split, its
    // partials requested 16 at a time before they are added in split order.
    __shared__ float wts[PF_MAX_SPLIT], wl[PF_MAX_SPLIT];
    const int row = blockIdx.x, t = row / a.H, d = threadIdx.x;
    const int ns = min(a.n_split, (a.p0 + t) / a.split_keys + 1);
    const float *p = a.part + (int64_t)row * a.n_split * (HD + 4);
    if (d < 64) {
        const int sl = min(d, ns - 1);
        const float ms = d < ns ? p[(int64_t)sl * (HD + 4)] : -INFINITY;
        const float ls = p[(int64_t)sl * (HD + 4) + 1];
        const float mx = wave_max(ms);
        const float w = ms == -INFINITY ? 0.f : exp2f(ms - mx);
        wts[d] = w, wl[d] = w * ls;
    }
    __syncthreads();
    float den = 0.f, num = 0.f;
    for (int s2 = 0; s2 < ns; s2++) den += wl[s2];
    for (int s0 = 0; s0 < ns; s0 += 16) {
        float o[16];
#pragma unroll
        for (int j = 0; j < 16; j++) o[j] = p[(int64_t)min(s0 + j, ns - 1) * (HD + 4) + 4 + d];
#pragma unroll
        for (int j = 0; j < 16; j++)
            if (s0 + j < ns) num += wts[s0 + j] * o[j];
    }
    a.out[(int64_t)row * HD + d] = num / den;
}

bool attn_prefill_supported(int H, int HKV, int HD) {
    if (HKV <= 0 || H % HKV) return false;
    const int G = H / HKV;
    return (HD == 64 || HD == 128) && G <= 64;
}

// Keys per split: a multiple of 64, at least 256, at most 16 splits, and
// no more splits than bring the launch to about 512 workgroups (wg: the
// workgroups of one split); every split adds (m, l, O) partials to merge.
static int pf_split_keys(int64_t max_keys, int64_t wg) {
    const int64_t splits = std::max<int64_t>(1, std::min<int64_t>(16, (512 + wg - 1) / wg));
    const int64_t per = std::max<int64_t>(256, (max_keys + splits - 1) / splits);
    return (int)((per + PF_KB - 1) / PF_KB * PF_KB);
}

// A bound for every launch with at most max_keys keys (splits <= 16 and
// <= max_keys / 256, both growing with the key count).
size_t attn_prefill_partial_bytes(int nq, int H, int HD, int64_t max_keys) {
    const int64_t ns = std::min<int64_t>(16, (max_keys + 255) / 256);
    return ns > 1 ? (size_t)nq * H * ns * (HD + 4) * sizeof(float) : 0;
}

hipError_t launch_attn_prefill(const float *q, int64_t q_stride, KvLayer kv, int kv_f16, int n_ctx, int H, int HKV,
                               int HD, int p0, int nq, float scale, float *part, float *out, hipStream_t s) {
    if (!attn_prefill_supported(H, HKV, HD) || nq < 1 || p0 < 0 || p0 + nq > n_ctx) return hipErrorInvalidValue;
    PfArgs a{};
    a.q = q, a.q_stride = q_stride, a.kv = kv, a.n_ctx = n_ctx, a.H = H, a.HKV = HKV, a.p0 = p0, a.nq = nq;
    a.scale = scale, a.part = part, a.out = out;
    const int64_t max_keys = (int64_t)p0 + nq;
    const int qb = PF_ROWS / (H / HKV);
    a.split_keys = pf_split_keys(max_keys, (int64_t)((nq + qb - 1) / qb) * HKV);
    a.n_split = (int)((max_keys + a.split_keys - 1) / a.split_keys);
    const int G = H / HKV, QB = PF_ROWS / G;
    const dim3 grid((unsigned)((nq + QB - 1) / QB), (unsigned)HKV, (unsigned)a.n_split);
    if (HD == 64) {
        if (kv_f16) hipLaunchKernelGGL((k_attn_pf<64, 0, true>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((k_attn_pf<64, 0, false>), grid, dim3(256), 0, s, a);
        if (a.n_split > 1) hipLaunchKernelGGL(k_attn_pf_merge<64>, dim3((unsigned)(nq * H)), dim3(64), 0, s, a);
        return hipGetLastError();
    }
    auto go = [&](auto fc) {
        constexpr bool F = decltype(fc)::value;
        switch (G) {
        case 1: hipLaunchKernelGGL((k_attn_pf<128, 1, F>), grid, dim3(256), 0, s, a); break;
        case 2: hipLaunchKernelGGL((k_attn_pf<128, 2, F>), grid, dim3(256), 0, s, a); break;
        case 4: hipLaunchKernelGGL((k_attn_pf<128, 4, F>), grid, dim3(256), 0, s, a); break;
        case 8: hipLaunchKernelGGL((k_attn_pf<128, 8, F>), grid, dim3(256), 0, s, a); break;
        default: hipLaunchKernelGGL((k_attn_pf<128, 0, F>), grid, dim3(256), 0, s, a); break;
        }
    };
    if (kv_f16) go(std::true_type{});
    else go(std::false_type{});
    if (a.n_split > 1) hipLaunchKernelGGL(k_attn_pf_merge<128>, dim3((unsigned)(nq * H)), dim3(128), 0, s, a);
    return hipGetLastError();
}

}  // namespace ts5hip
