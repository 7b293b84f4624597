// The k-quant matmul of several tokens: Y[t] = W x_t for t < M, reading each
// weight once per M tokens (engine/src/cpu_backend.cpp:18-41 at n > 1; the
// reference's GPU path uses mvt_q4_k / mvt_q6_k for 2..8 tokens and
// matmul_big for prompts, engine/src/vk_backend.cpp:835-918).
//
// Matrix cores. The activations are the same quantized form the one-token
// matvec reads (common.h Act: X = 65536*hi + 256*mid + lo, a scale per 32
// values), so every product is exact in integers and only the per-sub-block
// scaling runs in fp32. One v_mfma_i32_16x16x32_i8 multiplies 16 rows x 32
// weights (A: the raw quants, 0..15 or 0..63 or int8) by 32 values of 16
// tokens' hi plane (B), a second by their mid plane, a third by their lo
// plane; 65536*C_hi + 256*C_mid + C_lo is then sum q * X for each
// (row, token) of the sub-block, and
//   Q4_K: y += d*sc * xs * (sum q X) - dmin*m * (sum x)         per 32 values
//   Q6_K: y += d*sc * xs * (sum q X - 32 * sum X)              per 16 values
//   Q8_0: y += d * xs * (sum q X)                               per 32 values
// (engine/src/quants.cpp:133-202). Q6_K's 16-value groups each get MFMAs of
// their own, the other half of the 32-value A operand zeroed.
//
// Lane layout of the 16x16x32 int8 MFMA (checked on the device): A lane l =
// row l%16, k 8*(l/16)..+7; B lane l = column l%16, same k; D lane l holds
// rows 4*(l/16)+i (i = 0..3) of column l%16. A lane therefore loads 8 bytes
// of a row's quants and 8 bytes of a token's activation per sub-block, and
// needs the block scales of rows 4*(l/16)..+3, which lanes exchange through
// LDS (each lane decodes the scales of its own row and k-range).
//
// Workgroup: 4 waves, each 16 rows x 16*TN tokens; grid (rows/64, tokens /
// (16 TN), KS). With KS > 1 the blocks of a row are split over KS workgroups
// whose partial sums a second kernel adds in a fixed order.
#include <algorithm>
#include <cstdlib>
#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace ts5hip {
constexpr int GM_WAVES = 4;  // k_gemm_m's waves a workgroup, each a share of the row's blocks (8: 10 % slower)
constexpr int GM_RTMAX = 4;  // k_gemm_m's most 16-row tiles a wave
// Keeps the scheduler from moving loads or arithmetic across this point (the
// next item's weight requests stay ahead of the current item's arithmetic).
#define TS5_GM_SB() __builtin_amdgcn_sched_barrier(0)

typedef int v4i __attribute__((ext_vector_type(4)));
static int g_gemm_m_cu = 256;  // CUs, for k_gemm_m's row tiles a workgroup

struct GemmArgs {
    uint32_t t;
    const uint8_t *w, *w2;    // block bodies (w2: GLU's up projection)
    const uint16_t *s, *s2;   // split layouts' f16 block scales
    int nrows, nb, n_in, M, ks;
    const uint8_t *act;       // M activation records of gemm_act_bytes(t, n_in)
    int64_t act_stride;
    float *out;               // ks == 1: y [M][ldy]; ks > 1: partials [ks][2][M][nrows]
    const float *y_in;        // MODE_ADD: residual [M][ldy] (may be out)
    int64_t ldy;
    // k_gemm_m with its activation built in LDS (launch_gemm_fused): the fp32
    // input [M][xin_stride], rms-normalised by norm_w (may be null) first.
    const float *xin, *norm_w;
    int64_t xin_stride;
    float eps;
    // k_gemm_mx only: the outputs also as the next matmul's activation
    // records (mact_bytes(nrows) per token), row tiles then taken in pairs
    // (a 32-row chunk a workgroup; nrows a multiple of 256). Null: none.
    uint8_t *qout;
    int gelu;  // G_GLU: GELU (tanh form) for SiLU
};

enum { G_STORE = 0, G_ADD = 1, G_GLU = 2 };

__device__ inline uint64_t ld8(const void *p) { return *(const uint64_t *)p; }
__device__ inline uint4 ld16(const void *p) { return *(const uint4 *)p; }
__device__ inline v4i mfma(uint64_t a, uint64_t b) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8((long)a, (long)b, v4i{0, 0, 0, 0}, 0, 0, 0);
}
// The three planes' products of A with one B fragment, combined per entry:
// sum q X = 65536 C_hi + 256 C_mid + C_lo, in 64 bits (int8 or 6-bit quants
// can take the hi term past 2^31).
struct Prod3 {
    v4i c[3];
    __device__ long long at(int i) const { return (long long)c[0][i] * 65536 + c[1][i] * 256 + c[2][i]; }
};
__device__ inline Prod3 mfma3(uint64_t a, const uint64_t (&b)[3]) {
    Prod3 r;
#pragma unroll
    for (int P = 0; P < 3; P++) r.c[P] = mfma(a, b[P]);
    return r;
}

// Per-wave LDS for the scale exchange: [sub-block or group][row] (scale, min).
struct GemmLds {
    __align__(16) float2 scl[2][16][16];  // [matrix][sub-block / group][row]
};

// F_Q8M: the Q8SM layout (Q4_0, Q4_1, Q5_0, Q5_1, Q5_K), Q8_0's products plus
// a min per 32 values against the chunk's activation sum.
constexpr int F_Q4K = 0, F_Q6K = 1, F_Q80 = 2, F_Q8M = 3;
template <int FMT>
constexpr bool q8_rows = FMT == F_Q80 || FMT == F_Q8M;

// Activation fragments of token tok for 32-value chunk s of block b, k-group
// kq, and the chunk's scale and sum: Q4_K / Q6_K rows read the matmul layout
// (MACT_*), Q8_0 rows Act (its block is one chunk, s = 0).
struct AFrag {
    uint64_t p[3];  // planes hi, mid, lo
    float xs, xsum;
};
template <int FMT>
__device__ inline const uint8_t *mact_blk(const GemmArgs &a, int tok, int b) {
    return a.act + (int64_t)tok * a.act_stride + (int64_t)b * MACT_BLOCK;
}
template <int FMT>
__device__ inline AFrag act_frag(const GemmArgs &a, int tok, int b, int s, int kq) {
    AFrag f{{0, 0, 0}, 0.f, 0.f};
    if (tok < a.M) {
        if constexpr (q8_rows<FMT>) {
            const CAct x = cact_view(a.act + (int64_t)tok * a.act_stride, a.n_in);
            f.p[0] = ld8(x.hi + 32 * b + 8 * kq);
            f.p[1] = ld8(x.mid + 32 * b + 8 * kq);
            f.p[2] = ld8(x.lo + 32 * b + 8 * kq);
            f.xs = x.scale[b];
            f.xsum = x.sum[b];
        } else {
            const uint8_t *blk = mact_blk<FMT>(a, tok, b);
            f.p[0] = ld8(blk + 64 * kq + 8 * s);
            f.p[1] = ld8(blk + MACT_MID + 64 * kq + 8 * s);
            f.p[2] = ld8(blk + MACT_LO + 64 * kq + 8 * s);
            f.xs = ((const float *)(blk + MACT_SCALE))[s];
            f.xsum = ((const float *)(blk + MACT_SUM))[s];
        }
    }
    return f;
}

template <int FMT, int MODE, int TN>
__global__ __launch_bounds__(256) void k_gemm(GemmArgs a) {
    __shared__ GemmLds L[4];
    const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, kq = l >> 4, rl = l & 15;
    GemmLds &S = L[wave];
    const int r0 = blockIdx.x * 64 + wave * 16;
    const int t0 = blockIdx.y * 16 * TN;
    const int row = r0 + rl;                    // the row this lane loads quants / scales of
    const bool rin = row < a.nrows;
    const int bpk = (a.nb + a.ks - 1) / a.ks;  // blocks per split
    const int b0 = blockIdx.z * bpk, b1 = min(a.nb, b0 + bpk);
    constexpr int NW = MODE == G_GLU ? 2 : 1;
    float acc[NW][TN][4];
#pragma unroll
    for (int m = 0; m < NW; m++)
#pragma unroll
        for (int g = 0; g < TN; g++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[m][g][i] = 0.f;

    for (int b = b0; b < b1; b++) {
        __builtin_amdgcn_wave_barrier();  // this wave's reads of the last block's scales are issued
        if constexpr (q8_rows<FMT>) {
            uint64_t q[NW];
#pragma unroll
            for (int m = 0; m < NW; m++) {
                const int64_t blk = (int64_t)(rin ? row : 0) * a.nb + b;
                q[m] = rin ? ld8((m ? a.w2 : a.w) + blk * Q8_BODY + 8 * kq) : 0;
                if (kq == 0) {
                    if constexpr (FMT == F_Q8M)
                        S.scl[m][0][rl] = rin ? ((const float2 *)(m ? a.s2 : a.s))[blk] : make_float2(0.f, 0.f);
                    else
                        S.scl[m][0][rl] = make_float2(rin ? h2f((m ? a.s2 : a.s)[blk]) : 0.f, 0.f);
                }
            }
            __builtin_amdgcn_wave_barrier();
            AFrag x[TN];
#pragma unroll
            for (int g = 0; g < TN; g++) x[g] = act_frag<FMT>(a, t0 + 16 * g + rl, b, 0, kq);
#pragma unroll
            for (int m = 0; m < NW; m++) {
                const float4 sA = *(const float4 *)&S.scl[m][0][4 * kq];
                const float4 sB = *(const float4 *)&S.scl[m][0][4 * kq + 2];
                const float d[4] = {sA.x, sA.z, sB.x, sB.z}, mn[4] = {sA.y, sA.w, sB.y, sB.w};
#pragma unroll
                for (int g = 0; g < TN; g++) {
                    const Prod3 c = mfma3(q[m], x[g].p);
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        acc[m][g][i] += d[i] * x[g].xs * (float)c.at(i);
                        if constexpr (FMT == F_Q8M) acc[m][g][i] += mn[i] * x[g].xsum;
                    }
                }
            }
        } else {  // Q6_K
            uint64_t ql[NW][4], qh[NW][2];
#pragma unroll
            for (int m = 0; m < NW; m++) {
                const int64_t blk = (int64_t)(rin ? row : 0) * a.nb + b;
                const uint8_t *body = (m ? a.w2 : a.w) + blk * Q6K_BODY;
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    ql[m][2 * h] = rin ? ld8(body + 64 * h + 8 * kq) : 0;
                    ql[m][2 * h + 1] = rin ? ld8(body + 64 * h + 32 + 8 * kq) : 0;
                    qh[m][h] = rin ? ld8(body + 128 + 32 * h + 8 * kq) : 0;
                }
                const float d = rin ? h2f((m ? a.s2 : a.s)[blk]) : 0.f;
                const uint32_t scw = rin ? *(const uint32_t *)(body + 192 + 4 * kq) : 0;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    S.scl[m][4 * kq + j][rl] = make_float2(d * (float)(int8_t)((scw >> (8 * j)) & 0xff), 0.f);
            }
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int c32 = 0; c32 < 8; c32++) {  // 32-value chunk: half h = c32/4, quarter c = c32%4
                const int h = c32 >> 2, c = c32 & 3;
                AFrag x[TN];
                int is0[TN], is1[TN];
#pragma unroll
                for (int g = 0; g < TN; g++) {
                    const int tok = t0 + 16 * g + rl;
                    x[g] = act_frag<FMT>(a, tok, b, c32, kq);
                    is0[g] = is1[g] = 0;
                    if (tok < a.M) {
                        const int *isum = (const int *)(mact_blk<FMT>(a, tok, b) + MACT_ISUM);
                        is0[g] = isum[2 * c32];
                        is1[g] = isum[2 * c32 + 1];
                    }
                }
#pragma unroll
                for (int m = 0; m < NW; m++) {
                    const uint64_t lo4 = (ql[m][2 * h + (c & 1)] >> (4 * (c >> 1))) & 0x0F0F0F0F0F0F0F0Full;
                    const uint64_t hi2 = ((qh[m][h] >> (2 * c)) & 0x0303030303030303ull) << 4;
                    const uint64_t q = lo4 | hi2;  // 0..63
                    const uint64_t qa0 = kq < 2 ? q : 0, qa1 = kq < 2 ? 0 : q;
                    const int g0 = 2 * c32, g1 = 2 * c32 + 1;  // the block's 16-value groups
                    const float4 s0A = *(const float4 *)&S.scl[m][g0][4 * kq];
                    const float4 s0B = *(const float4 *)&S.scl[m][g0][4 * kq + 2];
                    const float4 s1A = *(const float4 *)&S.scl[m][g1][4 * kq];
                    const float4 s1B = *(const float4 *)&S.scl[m][g1][4 * kq + 2];
                    const float e0[4] = {s0A.x, s0A.z, s0B.x, s0B.z}, e1[4] = {s1A.x, s1A.z, s1B.x, s1B.z};
#pragma unroll
                    for (int g = 0; g < TN; g++) {
                        const Prod3 c0 = mfma3(qa0, x[g].p), c1 = mfma3(qa1, x[g].p);
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            acc[m][g][i] += x[g].xs * (e0[i] * (float)(c0.at(i) - 32ll * is0[g]) +
                                                       e1[i] * (float)(c1.at(i) - 32ll * is1[g]));
                    }
                }
                if constexpr (TN > 1) __builtin_amdgcn_sched_barrier(0);  // one chunk's loads at a time
            }
        }
    }

    // Results: rows r0 + 4*kq + i, tokens t0 + 16*g + rl.
#pragma unroll
    for (int g = 0; g < TN; g++) {
        const int tok = t0 + 16 * g + rl;
        if (tok >= a.M) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = r0 + 4 * kq + i;
            if (r >= a.nrows) continue;
            if (a.ks > 1) {
                float *p = a.out + (((int64_t)blockIdx.z * 2) * a.M + tok) * a.nrows + r;
                p[0] = acc[0][g][i];
                if (MODE == G_GLU) p[(int64_t)a.M * a.nrows] = acc[NW - 1][g][i];
            } else {
                const int64_t o = (int64_t)tok * a.ldy + r;
                const float v = acc[0][g][i];
                if (MODE == G_ADD) a.out[o] = a.y_in[o] + v;
                else if (MODE == G_GLU) a.out[o] = glu_act(v, acc[NW - 1][g][i], a.gelu);
                else a.out[o] = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Up to 16 tokens (the speculative verify batch): the matmul is a weight
// stream. A workgroup takes 16 rows; its 4 waves each take a quarter of the
// row's blocks and keep the next block's quants, header and activation
// fragments in flight while they compute the current one; the quarters' sums
// meet in LDS and are added in a fixed order.
// ---------------------------------------------------------------------------
template <int FMT, int NW>
struct WBlk {  // one block of the lane's row (rl) and k-group (kq), per matrix
    uint4 hdr[NW];     // Q4_K header
    uint64_t q[NW][4]; // Q4_K: the 4 nibble groups' 8 bytes; Q8_0: q[m][0]; Q6_K: ql (4)
    uint64_t qh[NW][2];
    uint32_t scw[NW];  // Q6_K: the 4 int8 scales of this k-group
    float d[NW];       // Q6_K / Q8_0 / Q8SM block scale
    float mn[NW];      // Q8SM block min
};

// Loads are unconditional (a row or token past the end reads the last one,
// then its scale is zeroed), so no branch separates a load from its use and
// the next block's loads stay in flight across the current block's compute.
template <int FMT, int NW>
__device__ inline WBlk<FMT, NW> load_wblk(const GemmArgs &a, int row, bool rin, int kq, int b) {
    WBlk<FMT, NW> w;
    const int64_t blk = (int64_t)min(row, a.nrows - 1) * a.nb + b;
#pragma unroll
    for (int m = 0; m < NW; m++) {
        const uint8_t *base = m ? a.w2 : a.w;
        if constexpr (FMT == F_Q4K) {
            const uint8_t *p = base + blk * Q4K_BYTES;
            w.hdr[m] = ld16(p);
#pragma unroll
            for (int g = 0; g < 4; g++) w.q[m][g] = ld8(p + 16 + 32 * g + 8 * kq);
        } else if constexpr (FMT == F_Q80) {
            w.q[m][0] = ld8(base + blk * Q8_BODY + 8 * kq);
            w.d[m] = h2f((m ? a.s2 : a.s)[blk]);
        } else if constexpr (FMT == F_Q8M) {
            w.q[m][0] = ld8(base + blk * Q8_BODY + 8 * kq);
            const float2 sm = ((const float2 *)(m ? a.s2 : a.s))[blk];
            w.d[m] = sm.x, w.mn[m] = sm.y;
        } else {
            const uint8_t *body = base + blk * Q6K_BODY;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                w.q[m][2 * h] = ld8(body + 64 * h + 8 * kq);
                w.q[m][2 * h + 1] = ld8(body + 64 * h + 32 + 8 * kq);
                w.qh[m][h] = ld8(body + 128 + 32 * h + 8 * kq);
            }
            w.scw[m] = *(const uint32_t *)(body + 192 + 4 * kq);
            w.d[m] = h2f((m ? a.s2 : a.s)[blk]);
        }
    }
    return w;
}

template <int FMT, int NW>
__device__ inline void mask_wblk(WBlk<FMT, NW> &w, bool rin) {
#pragma unroll
    for (int m = 0; m < NW; m++) {
        if constexpr (FMT == F_Q4K) w.hdr[m].x = rin ? w.hdr[m].x : 0u;  // d = dmin = 0
        else w.d[m] = rin ? w.d[m] : 0.f;
        if constexpr (FMT == F_Q8M) w.mn[m] = rin ? w.mn[m] : 0.f;
    }
}

// Activation fragments of one block for the lane's token and k-group.
template <int FMT>
struct ABlk {
    static constexpr int C = q8_rows<FMT> ? 1 : 8;  // 32-value chunks per block
    uint64_t p[C][3];  // [chunk][plane hi, mid, lo]
    float xs[C], xsum[C];
    int is[FMT == F_Q6K ? 16 : 1];
};

template <int FMT>
__device__ inline ABlk<FMT> load_ablk(const GemmArgs &a, int tok, int kq, int b) {
    ABlk<FMT> x;
    tok = min(tok, a.M - 1);
    if constexpr (q8_rows<FMT>) {
        const CAct xa = cact_view(a.act + (int64_t)tok * a.act_stride, a.n_in);
        x.p[0][0] = ld8(xa.hi + 32 * b + 8 * kq);
        x.p[0][1] = ld8(xa.mid + 32 * b + 8 * kq);
        x.p[0][2] = ld8(xa.lo + 32 * b + 8 * kq);
        x.xs[0] = xa.scale[b];
        x.xsum[0] = xa.sum[b];
    } else {  // the lane's 8 bytes of every chunk, side by side: 16-byte loads
        const uint8_t *blk = mact_blk<FMT>(a, tok, b);
#pragma unroll
        for (int c = 0; c < 8; c += 2) {
            const int plane[3] = {0, MACT_MID, MACT_LO};
#pragma unroll
            for (int P = 0; P < 3; P++) {
                const uint4 v = ld16(blk + plane[P] + 64 * kq + 8 * c);
                x.p[c][P] = ((uint64_t)v.y << 32) | v.x, x.p[c + 1][P] = ((uint64_t)v.w << 32) | v.z;
            }
        }
#pragma unroll
        for (int c = 0; c < 8; c += 4) {
            const float4 sc = *(const float4 *)(blk + MACT_SCALE + 4 * c);
            const float4 su = *(const float4 *)(blk + MACT_SUM + 4 * c);
            x.xs[c] = sc.x, x.xs[c + 1] = sc.y, x.xs[c + 2] = sc.z, x.xs[c + 3] = sc.w;
            x.xsum[c] = su.x, x.xsum[c + 1] = su.y, x.xsum[c + 2] = su.z, x.xsum[c + 3] = su.w;
        }
        if constexpr (FMT == F_Q6K) {
#pragma unroll
            for (int g = 0; g < 16; g += 4) {
                const int4 v = *(const int4 *)(blk + MACT_ISUM + 4 * g);
                x.is[g] = v.x, x.is[g + 1] = v.y, x.is[g + 2] = v.z, x.is[g + 3] = v.w;
            }
        }
    }
    return x;
}

template <int FMT>
__device__ inline void mask_ablk(ABlk<FMT> &x, bool tin) {
#pragma unroll
    for (int c = 0; c < ABlk<FMT>::C; c++) {
        x.xs[c] = tin ? x.xs[c] : 0.f;
        x.xsum[c] = tin ? x.xsum[c] : 0.f;
    }
}

// acc[m][i] += block b's products for rows 4*kq+i of the tile and token rl.
template <int FMT, int NW>
__device__ inline void compute_blk(GemmLds &S, const WBlk<FMT, NW> &w, const ABlk<FMT> &x, int kq, int rl,
                                   float (&acc)[NW][4]) {
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int m = 0; m < NW; m++) {
        if constexpr (FMT == F_Q4K) {
            int sc0, m0, sc1, m1;
            kq_scale_min_pair(kq, w.hdr[m].y, w.hdr[m].z, w.hdr[m].w, sc0, m0, sc1, m1);
            const float d = h2f(w.hdr[m].x & 0xffff), dmin = h2f(w.hdr[m].x >> 16);
            S.scl[m][2 * kq][rl] = make_float2(d * (float)sc0, dmin * (float)m0);
            S.scl[m][2 * kq + 1][rl] = make_float2(d * (float)sc1, dmin * (float)m1);
        } else if constexpr (q8_rows<FMT>) {
            if (kq == 0) S.scl[m][0][rl] = make_float2(w.d[m], FMT == F_Q8M ? w.mn[m] : 0.f);
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++)
                S.scl[m][4 * kq + j][rl] = make_float2(w.d[m] * (float)(int8_t)((w.scw[m] >> (8 * j)) & 0xff), 0.f);
        }
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int m = 0; m < NW; m++) {
        if constexpr (FMT == F_Q4K) {
#pragma unroll
            for (int s = 0; s < 8; s++) {
                const uint64_t qa = (s & 1) ? (w.q[m][s >> 1] >> 4) & 0x0F0F0F0F0F0F0F0Full
                                            : w.q[m][s >> 1] & 0x0F0F0F0F0F0F0F0Full;
                const float4 sA = *(const float4 *)&S.scl[m][s][4 * kq];
                const float4 sB = *(const float4 *)&S.scl[m][s][4 * kq + 2];
                const float dsc[4] = {sA.x, sA.z, sB.x, sB.z}, dm[4] = {sA.y, sA.w, sB.y, sB.w};
                v4i c[3];
#pragma unroll
                for (int P = 0; P < 3; P++) c[P] = mfma(qa, x.p[s][P]);
                // Exact in int32 for 4-bit quants: |.| <= 32 * 15 * (64 * 65536 + 128 * 257) < 2^31.
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[m][i] += dsc[i] * x.xs[s] * (float)(c[0][i] * 65536 + c[1][i] * 256 + c[2][i]) -
                                 dm[i] * x.xsum[s];
            }
        } else if constexpr (q8_rows<FMT>) {
            const float4 sA = *(const float4 *)&S.scl[m][0][4 * kq];
            const float4 sB = *(const float4 *)&S.scl[m][0][4 * kq + 2];
            const float d[4] = {sA.x, sA.z, sB.x, sB.z}, mn[4] = {sA.y, sA.w, sB.y, sB.w};
            const Prod3 c = mfma3(w.q[m][0], x.p[0]);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                acc[m][i] += d[i] * x.xs[0] * (float)c.at(i);
                if constexpr (FMT == F_Q8M) acc[m][i] += mn[i] * x.xsum[0];
            }
        } else {
#pragma unroll
            for (int c32 = 0; c32 < 8; c32++) {
                const int h = c32 >> 2, c = c32 & 3;
                const uint64_t lo4 = (w.q[m][2 * h + (c & 1)] >> (4 * (c >> 1))) & 0x0F0F0F0F0F0F0F0Full;
                const uint64_t hi2 = ((w.qh[m][h] >> (2 * c)) & 0x0303030303030303ull) << 4;
                const uint64_t q = lo4 | hi2;
                const uint64_t qa0 = kq < 2 ? q : 0, qa1 = kq < 2 ? 0 : q;
                const float4 s0A = *(const float4 *)&S.scl[m][2 * c32][4 * kq];
                const float4 s0B = *(const float4 *)&S.scl[m][2 * c32][4 * kq + 2];
                const float4 s1A = *(const float4 *)&S.scl[m][2 * c32 + 1][4 * kq];
                const float4 s1B = *(const float4 *)&S.scl[m][2 * c32 + 1][4 * kq + 2];
                const float e0[4] = {s0A.x, s0A.z, s0B.x, s0B.z}, e1[4] = {s1A.x, s1A.z, s1B.x, s1B.z};
                const Prod3 c0 = mfma3(qa0, x.p[c32]), c1 = mfma3(qa1, x.p[c32]);
#pragma unroll
                for (int i = 0; i < 4; i++)
                    acc[m][i] += x.xs[c32] * (e0[i] * (float)(c0.at(i) - 32ll * x.is[2 * c32]) +
                                                e1[i] * (float)(c1.at(i) - 32ll * x.is[2 * c32 + 1]));
            }
        }
    }
}

template <int FMT, int MODE>
__global__ __launch_bounds__(256) void k_gemm_small(GemmArgs a) {
    constexpr int NW = MODE == G_GLU ? 2 : 1;
    __shared__ GemmLds L[4];
    __shared__ float red[3][NW][64][4];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: a scalar block loop
    const int l = threadIdx.x & 63, kq = l >> 4, rl = l & 15;
    GemmLds &S = L[wave];
    const int r0 = blockIdx.x * 16, row = r0 + rl;
    const bool rin = row < a.nrows;
    const int bpq = (a.nb + 3) / 4, b0 = wave * bpq, b1 = min(a.nb, b0 + bpq);
    float acc[NW][4];
#pragma unroll
    for (int m = 0; m < NW; m++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[m][i] = 0.f;
    const bool tin = rl < a.M;
    if (b0 < b1) {  // ping-pong buffers: no register copy waits on a load in flight
        WBlk<FMT, NW> wA = load_wblk<FMT, NW>(a, row, rin, kq, b0), wB;
        ABlk<FMT> xA = load_ablk<FMT>(a, rl, kq, b0), xB;
        for (int b = b0;;) {
            wB = load_wblk<FMT, NW>(a, row, rin, kq, min(b + 1, b1 - 1));
            xB = load_ablk<FMT>(a, rl, kq, min(b + 1, b1 - 1));
            mask_wblk(wA, rin), mask_ablk(xA, tin);
            compute_blk<FMT, NW>(S, wA, xA, kq, rl, acc);
            if (++b >= b1) break;
            wA = load_wblk<FMT, NW>(a, row, rin, kq, min(b + 1, b1 - 1));
            xA = load_ablk<FMT>(a, rl, kq, min(b + 1, b1 - 1));
            mask_wblk(wB, rin), mask_ablk(xB, tin);
            compute_blk<FMT, NW>(S, wB, xB, kq, rl, acc);
            if (++b >= b1) break;
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int m = 0; m < NW; m++)
#pragma unroll
            for (int i = 0; i < 4; i++) red[wave - 1][m][l][i] = acc[m][i];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int q = 0; q < 3; q++)
#pragma unroll
        for (int m = 0; m < NW; m++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[m][i] += red[q][m][l][i];
    const int tok = rl;
    if (tok >= a.M) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = r0 + 4 * kq + i;
        if (r >= a.nrows) continue;
        const int64_t o = (int64_t)tok * a.ldy + r;
        const float v = acc[0][i];
        if (MODE == G_ADD) a.out[o] = a.y_in[o] + v;
        else if (MODE == G_GLU) a.out[o] = glu_act(v, acc[NW - 1][i], a.gelu);
        else a.out[o] = v;
    }
}

// ---------------------------------------------------------------------------
// Q4_K rows, up to 8 tokens (k_gemm_m): the roles of the MFMA operands
// swapped so that each lane's result is one (token, row) pair. A = 16
// activation rows, 4 tokens x 4 planes (hi, mid, lo, and an unused fourth), of a
// 32-value sub-block; B = the sub-block's quants of 16 weight rows. D lane l
// then holds the 4 planes of token l/16 for weight row l%16, so
// 65536 C_hi + 256 C_mid + C_lo and the block scaling
//   y += d*sc * xs * (sum q X) - dmin*m * (sum x)       (quants.cpp:140-157)
// happen in the lane, every lane holding a pair of the output. NT (1 or 2)
// tiles of 4 tokens, RT tiles of 16 rows a workgroup; the 4 waves split each row's
// blocks in quarters, and a wave keeps a block's activation fragments while it
// walks the RT row tiles (weights one item ahead), so the activation is read
// once per block and row group. The quarters meet in LDS in a fixed order.
// ---------------------------------------------------------------------------
template <int FMT, int NT, bool P5>
struct MAFrag {
    static constexpr int NQ = FMT == F_Q6K ? NT : 1, NQ4 = FMT == F_Q6K && P5 ? 16 : 1;
    uint64_t p[NT][8];          // A: [token tile][sub-block] 8 bytes of plane (l%16)%4 of token (l%16)/4
    float xs[NT][8], xsum[NT][8];  // epilogue token l/16 of each tile: scale, sum per sub-block
    float xs4[P5 ? 8 : 1], xsum4[P5 ? 8 : 1];  // P5: the fifth token's scales and sums
    int is[NQ][16], is4[NQ4];  // Q6_K: sum of X per 16 values (the -32 offset of its quants)
};
template <int FMT, int NW>
struct MWFrag;
template <int NW>
struct MWFrag<F_Q4K, NW> {
    uint4 hdr[NW];
    uint64_t q[NW][4];  // B: the lane's k-group bytes of the 4 nibble groups of row l%16
};
template <int NW>
struct MWFrag<F_Q6K, NW> {
    uint64_t ql[NW][2][2], qh[NW][2];  // per half: ql bytes 8kq.. and 32 + 8kq.., qh bytes 8kq..
    uint4 sc[NW];                      // the row's 16 int8 scales
    float d[NW];
};

template <int FMT, int NT, bool P5>
__device__ inline void load_mafrag_at(const uint8_t *act, int64_t act_stride, int M, int b, int l,
                                      MAFrag<FMT, NT, P5> &f);
template <int FMT, int NT, bool P5>
__device__ inline void load_mafrag(const GemmArgs &a, int b, int l, MAFrag<FMT, NT, P5> &f) {
    load_mafrag_at<FMT, NT, P5>(a.act, a.act_stride, a.M, b, l, f);
}
// The records of M tokens at act (global memory, or a workgroup's LDS copy).
template <int FMT, int NT, bool P5>
__device__ inline void load_mafrag_at(const uint8_t *act, int64_t act_stride, int M, int b, int l,
                                      MAFrag<FMT, NT, P5> &f) {
    const int kq = l >> 4, ar = l & 15, at = ar >> 2, ap = ar & 3, et = kq;
    // Row plane 3 of the A tile repeats the lo plane: its D row is computed
    // and never read (the combine takes planes 0-2), so the loaded values go
    // to the MFMA untouched and nothing here waits for them. With P5 (five
    // tokens in one tile) row 4t + 3 carries plane t of the fifth token
    // instead (t < 3; row 15 repeats its lo plane, unused).
    const int plane_of = P5 && ap == 3 ? min(at, 2) : ap;
    const int plane = plane_of == 0 ? 0 : plane_of == 1 ? MACT_MID : MACT_LO;
#pragma unroll
    for (int tt = 0; tt < NT; tt++) {
        const int tok = P5 && ap == 3 ? 4 : min(4 * tt + at, M - 1);
        const uint8_t *blk = act + (int64_t)tok * act_stride + (int64_t)b * MACT_BLOCK + plane + 64 * kq;
#pragma unroll
        for (int s2 = 0; s2 < 8; s2 += 2) {
            const uint4 v = ld16(blk + 8 * s2);
            f.p[tt][s2] = ((uint64_t)v.y << 32) | v.x;
            f.p[tt][s2 + 1] = ((uint64_t)v.w << 32) | v.z;
        }
        const int etok = min(4 * tt + et, M - 1);
        const uint8_t *eb = act + (int64_t)etok * act_stride + (int64_t)b * MACT_BLOCK;
#pragma unroll
        for (int c = 0; c < 8; c += 4) {
            const float4 sc = *(const float4 *)(eb + MACT_SCALE + 4 * c);
            f.xs[tt][c] = sc.x, f.xs[tt][c + 1] = sc.y, f.xs[tt][c + 2] = sc.z, f.xs[tt][c + 3] = sc.w;
            if constexpr (FMT == F_Q4K) {
                const float4 su = *(const float4 *)(eb + MACT_SUM + 4 * c);
                f.xsum[tt][c] = su.x, f.xsum[tt][c + 1] = su.y, f.xsum[tt][c + 2] = su.z, f.xsum[tt][c + 3] = su.w;
            }
        }
        if constexpr (FMT == F_Q6K)
#pragma unroll
            for (int c = 0; c < 16; c += 4) {
                const int4 v = *(const int4 *)(eb + MACT_ISUM + 4 * c);
                f.is[tt][c] = v.x, f.is[tt][c + 1] = v.y, f.is[tt][c + 2] = v.z, f.is[tt][c + 3] = v.w;
            }
    }
    if constexpr (P5) {
        const uint8_t *eb = act + 4 * act_stride + (int64_t)b * MACT_BLOCK;
#pragma unroll
        for (int c = 0; c < 8; c += 4) {
            const float4 sc = *(const float4 *)(eb + MACT_SCALE + 4 * c);
            f.xs4[c] = sc.x, f.xs4[c + 1] = sc.y, f.xs4[c + 2] = sc.z, f.xs4[c + 3] = sc.w;
            if constexpr (FMT == F_Q4K) {
                const float4 su = *(const float4 *)(eb + MACT_SUM + 4 * c);
                f.xsum4[c] = su.x, f.xsum4[c + 1] = su.y, f.xsum4[c + 2] = su.z, f.xsum4[c + 3] = su.w;
            }
        }
        if constexpr (FMT == F_Q6K)
#pragma unroll
            for (int c = 0; c < 16; c += 4) {
                const int4 v = *(const int4 *)(eb + MACT_ISUM + 4 * c);
                f.is4[c] = v.x, f.is4[c + 1] = v.y, f.is4[c + 2] = v.z, f.is4[c + 3] = v.w;
            }
    }
}

template <int FMT, int NW>
__device__ inline void load_mwfrag(const GemmArgs &a, int row, int kq, int b, MWFrag<FMT, NW> &w) {
    const int64_t blk = (int64_t)min(row, a.nrows - 1) * a.nb + b;
#pragma unroll
    for (int m = 0; m < NW; m++) {
        if constexpr (FMT == F_Q4K) {
            const uint8_t *p = (m ? a.w2 : a.w) + blk * Q4K_BYTES;
            w.hdr[m] = ld16(p);
#pragma unroll
            for (int g = 0; g < 4; g++) w.q[m][g] = ld8(p + 16 + 32 * g + 8 * kq);
        } else {
            const uint8_t *body = (m ? a.w2 : a.w) + blk * Q6K_BODY;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                w.ql[m][h][0] = ld8(body + 64 * h + 8 * kq);
                w.ql[m][h][1] = ld8(body + 64 * h + 32 + 8 * kq);
                w.qh[m][h] = ld8(body + 128 + 32 * h + 8 * kq);
            }
            w.sc[m] = ld16(body + 192);
            w.d[m] = h2f((m ? a.s2 : a.s)[blk]);
        }
    }
}

// P5: lane group kq holds plane kq of the fifth token; its scales are taken
// times that plane's weight in X (65536, 256, 1; 0 for the unused fourth),
// and its sums times 1 in group 0 only (the min term once), once per block
// rather than per item: the weights are powers of two or 0 and 1, so the
// products are exact and the results those of applying them per item.
template <int FMT, int NT, bool P5>
__device__ inline void gm_prescale(MAFrag<FMT, NT, P5> &x, int kq) {
    if constexpr (P5) {
        const float pw = kq == 0 ? 65536.f : kq == 1 ? 256.f : kq == 2 ? 1.f : 0.f;
        const float mw = kq == 0 ? 1.f : 0.f;
#pragma unroll
        for (int s8 = 0; s8 < 8; s8++) {
            x.xs4[s8] *= pw;
            if constexpr (FMT == F_Q4K) x.xsum4[s8] *= mw;
        }
    }
}

// One item of k_gemm_m / k_gemm_mx: block b of a row tile of 16 rows, the
// lane's row (rin: the row exists) and token planes; every MFMA of the
// item, then the scaling into acc (per matrix, per token tile).
template <int FMT, int NW, int NT, bool P5, int NA>
__device__ inline void gm_item(const MWFrag<FMT, NW> &w, const MAFrag<FMT, NT, P5> &x, float (&acc)[NW][NA], bool rin,
                               int kq) {
    if constexpr (FMT == F_Q6K) {
        constexpr uint64_t M0F = 0x0F0F0F0F0F0F0F0Full, M30 = 0x3030303030303030ull, M80 = 0x8080808080808080ull,
                           M20 = 0x2020202020202020ull;
        const uint64_t mlo = kq < 2 ? ~0ull : 0ull;  // lane groups 0-1 hold values 0-15 of a chunk
#pragma unroll
        for (int m = 0; m < NW; m++) {
            const float d = rin ? w.d[m] : 0.f;
            const uint32_t scw[4] = {w.sc[m].x, w.sc[m].y, w.sc[m].z, w.sc[m].w};
#pragma unroll
            for (int h = 0; h < 2; h++) {
                const uint64_t qa = w.ql[m][h][0], qb = w.ql[m][h][1], qh = w.qh[m][h];
                const uint64_t q[4] = {(qa & M0F) | ((qh << 4) & M30), (qb & M0F) | ((qh << 2) & M30),
                                       ((qa >> 4) & M0F) | (qh & M30), ((qb >> 4) & M0F) | ((qh >> 2) & M30)};
                v4i c[4][2];
#pragma unroll
                for (int cq = 0; cq < 4; cq++) {
                    const uint64_t qc = ((q[cq] | M80) - M20) ^ M80;  // q - 32 per byte
                    c[cq][0] = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)x.p[0][4 * h + cq], (long)(qc & mlo),
                                                                     v4i{0, 0, 0, 0}, 0, 0, 0);
                    c[cq][1] = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)x.p[0][4 * h + cq], (long)(qc & ~mlo),
                                                                     v4i{0, 0, 0, 0}, 0, 0, 0);
                }
#pragma unroll
                for (int cq = 0; cq < 4; cq++)
#pragma unroll
                    for (int g = 0; g < 2; g++) {
                        const int si = 8 * h + 2 * cq + g;
                        const float ds = d * (float)(int8_t)(scw[si >> 2] >> (8 * (si & 3)));
                        // |65536 C_hi| <= 2^31 (exact in fp32), |256 C_mid + C_lo| <= 2^24 + 2^16.
                        const float v = (float)c[cq][g][0] * 65536.f + (float)(c[cq][g][1] * 256 + c[cq][g][2]);
                        acc[m][0] += ds * x.xs[0][4 * h + cq] * v;
                        if constexpr (P5) acc[m][1] += ds * x.xs4[4 * h + cq] * (float)c[cq][g][3];
                    }
            }
        }
    } else {
#pragma unroll
        for (int m = 0; m < NW; m++) {
            const float d = rin ? h2f(w.hdr[m].x & 0xffff) : 0.f, dmin = rin ? h2f(w.hdr[m].x >> 16) : 0.f;
            float dsc[8], dm[8];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                int sc0, m0, sc1, m1;
                kq_scale_min_pair(g, w.hdr[m].y, w.hdr[m].z, w.hdr[m].w, sc0, m0, sc1, m1);
                dsc[2 * g] = d * (float)sc0, dm[2 * g] = dmin * (float)m0;
                dsc[2 * g + 1] = d * (float)sc1, dm[2 * g + 1] = dmin * (float)m1;
            }
            // Every MFMA of the item first, the scaling after: the results are
            // not waited for one at a time.
            v4i c[8][NT];
#pragma unroll
            for (int s8 = 0; s8 < 8; s8++) {
                const uint64_t qb = (s8 & 1) ? (w.q[m][s8 >> 1] >> 4) & 0x0F0F0F0F0F0F0F0Full
                                             : w.q[m][s8 >> 1] & 0x0F0F0F0F0F0F0F0Full;
#pragma unroll
                for (int tt = 0; tt < NT; tt++)
                    c[s8][tt] = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)x.p[tt][s8], (long)qb, v4i{0, 0, 0, 0}, 0, 0, 0);
            }
#pragma unroll
            for (int s8 = 0; s8 < 8; s8++)
#pragma unroll
                for (int tt = 0; tt < NT; tt++) {
                    // Exact in int32 for 4-bit quants: |.| <= 32 * 15 * (64 * 65536 + 128 * 257) < 2^31.
                    const int v = c[s8][tt][0] * 65536 + c[s8][tt][1] * 256 + c[s8][tt][2];
                    acc[m][tt] += dsc[s8] * x.xs[tt][s8] * (float)v - dm[s8] * x.xsum[tt][s8];
                }
            if constexpr (P5) {
#pragma unroll
                for (int s8 = 0; s8 < 8; s8++)
                    acc[m][NT] += dsc[s8] * x.xs4[s8] * (float)c[s8][0][3] - dm[s8] * x.xsum4[s8];
            }
        }
    }
}

// TM: 1 (up to 4 tokens, one A tile), 2 (5-8 tokens, two tiles) or 5
// (exactly 5 tokens in one tile: rows 4t + 3 carry the fifth token's planes,
// one per lane group, so D lane group t holds the fifth token's plane t for
// its row; each lane accumulates its plane's share of the fifth token,
// weighted by 65536 / 256 / 1, and the four groups' shares are added once at
// the end). A verify batch is the pending token and 4 drafts: 5 tokens.
// Q6_K rows (FMT F_Q6K; one A tile: TM 1 or 5): the quants enter B centred,
// q - 32 as int8 ((q | 0x80) - 0x20, then bit 7 flipped, per byte with no
// borrow between bytes), and each 32-value chunk takes two MFMAs, B's values
// 0-15 (lane groups 0-1) and 16-31 (groups 2-3) apart, for the two int8
// scales of 16 values: y += d * sc * xs * sum (q - 32) X (quants.cpp:179-202).
//
// XL (Q4_K, up to 5 tokens, n_in <= 4096): the workgroup builds the tokens'
// activation records itself, in LDS, from the fp32 input (one 16-value run a
// thread per token, rms-normalised first when norm_w is given), while its
// first weights are in flight, instead of a separate quantization launch
// writing them to HBM; the items then read their fragments from LDS.
template <int FMT, int MODE, int TM, int RT, bool XL = false>
__global__ __launch_bounds__(64 * GM_WAVES) void k_gemm_m(GemmArgs a) {
    constexpr int NW = MODE == G_GLU ? 2 : 1, NT = TM == 2 ? 2 : 1;
    constexpr bool P5 = TM == 5;
    static_assert(FMT == F_Q4K || NT == 1, "Q6_K rows: up to 5 tokens");
    constexpr int NA = NT + (P5 ? 1 : 0);  // accumulators per (row tile, matrix): tiles, then the fifth token
    __shared__ float red[GM_WAVES - 1][RT][NW][NA][64];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l = threadIdx.x & 63, kq = l >> 4, rl = l & 15;
    const int r0 = blockIdx.x * 16 * RT;
    const int bpq = (a.nb + GM_WAVES - 1) / GM_WAVES, b0 = wave * bpq, b1 = min(a.nb, b0 + bpq);
    float acc[RT][NW][NA];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int m = 0; m < NW; m++)
#pragma unroll
            for (int tt = 0; tt < NA; tt++) acc[r][m][tt] = 0.f;
    auto compute = [&](const MWFrag<FMT, NW> &w, const MAFrag<FMT, NT, P5> &x, int r) {
        gm_item<FMT, NW, NT, P5, NA>(w, x, acc[r], r0 + 16 * r + rl < a.nrows, kq);
    };
    auto prescale = [&](MAFrag<FMT, NT, P5> &x) { gm_prescale<FMT, NT, P5>(x, kq); };
    if constexpr (XL) {
        static_assert(FMT == F_Q4K && NT == 1 && GM_WAVES == 4, "fused activation: Q4_K, up to 5 tokens");
        extern __shared__ __align__(16) uint8_t lx[];  // [M][nb] activation records
        __shared__ float ssr[5][GM_WAVES];
        constexpr int MT = P5 ? 5 : 4;  // token slots read (past a.M: repeats, not used)
        const int nr = a.n_in / 16, run = min((int)threadIdx.x, nr - 1);
        const int64_t tstride = (int64_t)a.nb * MACT_BLOCK;
        // The input runs first (loads return in order), then the first item's
        // weights, all unconditional: rows, blocks and runs are clamped.
        float4 xv[MT][4], nw[4];
        const float *nwp = a.norm_w ? a.norm_w : a.xin;
#pragma unroll
        for (int t = 0; t < MT; t++)
#pragma unroll
            for (int j = 0; j < 4; j++)
                xv[t][j] = *(const float4 *)(a.xin + (int64_t)min(t, a.M - 1) * a.xin_stride + 16 * run + 4 * j);
#pragma unroll
        for (int j = 0; j < 4; j++) nw[j] = *(const float4 *)(nwp + 16 * run + 4 * j);
        MWFrag<FMT, NW> wA, wB;
        load_mwfrag<FMT, NW>(a, r0 + rl, kq, min(b0, a.nb - 1), wA);
        const bool mine = (int)threadIdx.x < nr;
        float sc[MT];
#pragma unroll
        for (int t = 0; t < MT; t++) sc[t] = 1.f;
        if (a.norm_w) {  // engine/src/cpu_backend.cpp:48-53, per token
#pragma unroll
            for (int t = 0; t < MT; t++) {
                float ss = 0.f;
#pragma unroll
                for (int j = 0; j < 4; j++)
                    ss += xv[t][j].x * xv[t][j].x + xv[t][j].y * xv[t][j].y + xv[t][j].z * xv[t][j].z +
                          xv[t][j].w * xv[t][j].w;
                ss = wave_sum_dpp(mine ? ss : 0.f);
                if (l == 0) ssr[t][wave] = ss;
            }
            __syncthreads();
#pragma unroll
            for (int t = 0; t < MT; t++) {
                float ss = 0.f;
#pragma unroll
                for (int w = 0; w < GM_WAVES; w++) ss += ssr[t][w];
                sc[t] = 1.0f / sqrtf(ss / (float)a.n_in + a.eps);
            }
        }
#pragma unroll
        for (int t = 0; t < MT; t++) {
            float v[16];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 f = xv[t][j], g = nw[j];
                v[4 * j] = f.x, v[4 * j + 1] = f.y, v[4 * j + 2] = f.z, v[4 * j + 3] = f.w;
                if (a.norm_w) {
                    v[4 * j] = v[4 * j] * sc[t] * g.x, v[4 * j + 1] = v[4 * j + 1] * sc[t] * g.y;
                    v[4 * j + 2] = v[4 * j + 2] * sc[t] * g.z, v[4 * j + 3] = v[4 * j + 3] * sc[t] * g.w;
                }
            }
            // quant_run_m pairs adjacent lanes (runs 2g, 2g + 1): nr is a
            // multiple of 16, so both or neither are `mine`.
            if (t < a.M && mine) quant_run_m(v, run, lx + t * tstride);
        }
        __syncthreads();
        wait_vmcnt<5 * NW>();  // the input loads are in: only the first item's weights may be open
        // Items (block b, row tile r) through the two weight buffers in turn,
        // each block's activation fragments read from LDS once.
        auto run_block = [&](auto par, int b) {
            constexpr int P = decltype(par)::value;
            MAFrag<FMT, NT, P5> xc;
            load_mafrag_at<FMT, NT, P5>(lx, tstride, a.M, b, l, xc);
            prescale(xc);
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const bool last = r == RT - 1;
                const int nb2 = last ? min(b + 1, b1 - 1) : b, nr2 = last ? 0 : r + 1;
                if ((P + r) & 1) {
                    load_mwfrag<FMT, NW>(a, r0 + 16 * nr2 + rl, kq, nb2, wA);
                    TS5_GM_SB();
                    compute(wB, xc, r);
                } else {
                    load_mwfrag<FMT, NW>(a, r0 + 16 * nr2 + rl, kq, nb2, wB);
                    TS5_GM_SB();
                    compute(wA, xc, r);
                }
            }
        };
        if (b0 < b1)
            for (int b = b0;; b += 2) {
                run_block(std::integral_constant<int, 0>{}, b);
                if (b + 1 >= b1) break;
                run_block(std::integral_constant<int, RT & 1>{}, b + 1);
                if (b + 2 >= b1) break;
            }
    } else if (b0 < b1) {
        MAFrag<FMT, NT, P5> xA, xB;
        MWFrag<FMT, NW> wA, wB;
        // In the order the loop requests them (weights, then activation), so
        // that the loop starts in the state its back edge brings.
        load_mwfrag<FMT, NW>(a, r0 + rl, kq, b0, wA);
        load_mafrag<FMT, NT, P5>(a, b0, l, xA);
        // Items (block b, row tile r) in order through two weight buffers in
        // turn, the blocks' activation fragments through two more: an item
        // first requests the next item's weights (at a block's last tile also
        // the next block's activation), unconditionally (past the last item a
        // repeat, in bounds and not used), then computes. No branch sits
        // between a request and the arithmetic after it, so the compiler's
        // waits for this item leave the next one's loads in flight (a request
        // under a branch made it wait for everything, vmcnt(0)).
        auto run_block = [&](auto par, int b, MAFrag<FMT, NT, P5> &xc, MAFrag<FMT, NT, P5> &xn) {
            constexpr int P = decltype(par)::value;
#pragma unroll
            for (int r = 0; r < RT; r++) {
                const bool last = r == RT - 1;
                const int nb2 = last ? min(b + 1, b1 - 1) : b, nr = last ? 0 : r + 1;
                // sched_barrier: the scheduler would otherwise sink the requests
                // below the arithmetic (register pressure) and lose the overlap.
                if ((P + r) & 1) {
                    load_mwfrag<FMT, NW>(a, r0 + 16 * nr + rl, kq, nb2, wA);
                    if (last) load_mafrag<FMT, NT, P5>(a, nb2, l, xn);
                    TS5_GM_SB();
                    if (r == 0) prescale(xc);
                    compute(wB, xc, r);
                } else {
                    load_mwfrag<FMT, NW>(a, r0 + 16 * nr + rl, kq, nb2, wB);
                    if (last) load_mafrag<FMT, NT, P5>(a, nb2, l, xn);
                    TS5_GM_SB();
                    if (r == 0) prescale(xc);
                    compute(wA, xc, r);
                }
            }
        };
        for (int b = b0;; b += 2) {
            run_block(std::integral_constant<int, 0>{}, b, xA, xB);
            if (b + 1 >= b1) break;
            run_block(std::integral_constant<int, RT & 1>{}, b + 1, xB, xA);
            if (b + 2 >= b1) break;
        }
    }
    if (wave > 0) {
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int m = 0; m < NW; m++)
#pragma unroll
                for (int tt = 0; tt < NA; tt++) red[wave - 1][r][m][tt][l] = acc[r][m][tt];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int q = 0; q < GM_WAVES - 1; q++)
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int m = 0; m < NW; m++)
#pragma unroll
                for (int tt = 0; tt < NA; tt++) acc[r][m][tt] += red[q][r][m][tt][l];
    if constexpr (P5)  // the four lane groups' shares of the fifth token, in every lane
#pragma unroll
        for (int r = 0; r < RT; r++)
#pragma unroll
            for (int m = 0; m < NW; m++) acc[r][m][NT] = add_xor32(add_xor16(acc[r][m][NT]));
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const int row = r0 + 16 * r + rl;
#pragma unroll
        for (int tt = 0; tt < NA; tt++) {
            const int tok = tt == NT ? 4 : 4 * tt + kq;  // the fifth token: written by lane group 0
            if (row >= a.nrows || tok >= a.M || (tt == NT && kq != 0)) continue;
            const int64_t o = (int64_t)tok * a.ldy + row;
            const float v = acc[r][0][tt];
            if (MODE == G_ADD) a.out[o] = a.y_in[o] + v;
            else if (MODE == G_GLU) a.out[o] = glu_act(v, acc[r][NW - 1][tt], a.gelu);
            else a.out[o] = v;
        }
    }
}

template <int FMT, int MODE, int TM>
static void launch_gemm_m_nt(const GemmArgs &a, int rt, hipStream_t s) {
    const unsigned grid = (unsigned)((a.nrows + 16 * rt - 1) / (16 * rt));
    if (rt == 4) hipLaunchKernelGGL((k_gemm_m<FMT, MODE, TM, 4>), dim3(grid), dim3(64 * GM_WAVES), 0, s, a);
    else if (rt == 2) hipLaunchKernelGGL((k_gemm_m<FMT, MODE, TM, 2>), dim3(grid), dim3(64 * GM_WAVES), 0, s, a);
    else hipLaunchKernelGGL((k_gemm_m<FMT, MODE, TM, 1>), dim3(grid), dim3(64 * GM_WAVES), 0, s, a);
}

// ---------------------------------------------------------------------------
// The fused small-batch matmul (Q4_K, 1-5 tokens, inputs up to 4096 wide:
// launch_gemm_fused) as one workgroup of 8 waves a CU. The workgroup builds
// the tokens' activation records in LDS once, from the fp32 input (norm
// fused), its threads in two halves of 256 with a token's 16-value runs to
// one half, and then takes RT row tiles of 16 rows, gridDim.x tiles apart
// (tile blockIdx.x + r * gridDim.x; past the last tile its loads repeat the
// last row and add nothing), each wave an eighth of every tile's blocks, the
// weights one item ahead. The waves' sums then meet in LDS and each thread
// finishes one (row tile, token tile, lane) entry, adding the waves in
// order. Against one workgroup of 4 waves per row tile (k_gemm_m's XL path)
// the activation is built once a CU, not once a tile, and never by two
// workgroups sharing a CU's SIMDs: that build is the VALU work the kernel
// repeats most.
// ---------------------------------------------------------------------------
constexpr int GX_WAVES = 8;

template <int MODE, int TM, int RT>
__global__ __launch_bounds__(64 * GX_WAVES) void k_gemm_mx(GemmArgs a) {
    constexpr int FMT = F_Q4K, NW = MODE == G_GLU ? 2 : 1, NT = 1;
    constexpr bool P5 = TM == 5;
    static_assert(TM == 1 || TM == 5, "fused small-batch matmul: up to 5 tokens");
    constexpr int NA = NT + (P5 ? 1 : 0);
    constexpr int MT = P5 ? 5 : 4;      // token slots read (past a.M: repeats, not used)
    constexpr int TH = (MT + 1) / 2;    // token slots of a half of the threads (the second half: MT - TH)
    extern __shared__ __align__(16) uint8_t lx[];  // [M][nb] activation records, then the waves' sums
    __shared__ float ssr[MT][4];
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l = tid & 63, kq = l >> 4, rl = l & 15;
    const int bpq = (a.nb + GX_WAVES - 1) / GX_WAVES, b0 = wave * bpq, b1 = min(a.nb, b0 + bpq);
    const int64_t tstride = (int64_t)a.nb * MACT_BLOCK;
    // An item's weights (16 rows x 144 bytes of one block, per matrix) come
    // into the wave's own LDS slot by DMA as row-contiguous 16-byte pieces
    // (piece c = 64 i + lane of request i: row c / 9, bytes 16 (c % 9); the
    // third request's first 16 lanes end the 144 pieces), two slots in turn,
    // one item ahead; the MFMA lanes then read their fragments from LDS.
    // Requested so, the bytes stream at about 1.7 times the rate of each
    // lane fetching its own 8-byte pieces of 16 rows from memory.
    constexpr int WSLOT = 16 * Q4K_BYTES;
    uint8_t *stg = lx + (size_t)a.M * tstride + (size_t)wave * 2 * NW * WSLOT;
    const uint32_t wbytes = (uint32_t)a.nrows * a.nb * Q4K_BYTES;  // rows past the last read zeros
    const __amdgpu_buffer_rsrc_t rw[2] = {buf_rsrc(a.w, wbytes), buf_rsrc(NW == 2 ? a.w2 : a.w, wbytes)};
    uint32_t coff[3];
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const int c = min(64 * i + l, 143);
        coff[i] = (uint32_t)((c / 9) * a.nb * Q4K_BYTES + 16 * (c % 9));
    }
    auto issue = [&](int row0, int b, int slot) {
        uint32_t base = ((uint32_t)row0 * a.nb + b) * Q4K_BYTES;
        asm volatile("" : "+s"(base));  // opaque: the per-lane sums are formed here, not hoisted out of the loop
#pragma unroll
        for (int m = 0; m < NW; m++)
#pragma unroll
            for (int i = 0; i < 3; i++)
                if (i < 2 || l < 16) dma16b(rw[m], base + coff[i], lds_addr(stg + (slot * NW + m) * WSLOT + 1024 * i));
    };
    auto fetch = [&](int slot, MWFrag<FMT, NW> &w) {
#pragma unroll
        for (int m = 0; m < NW; m++) {
            const uint8_t *p = stg + (slot * NW + m) * WSLOT + Q4K_BYTES * rl;
            w.hdr[m] = *(const uint4 *)p;
#pragma unroll
            for (int g = 0; g < 4; g++) w.q[m][g] = *(const uint64_t *)(p + 16 + 32 * g + 8 * kq);
        }
    };
    // Row tile r of the workgroup: tile blockIdx.x + r gridDim.x, or with
    // qout, tile 2 p + (r & 1) of pair p = blockIdx.x + (r / 2) gridDim.x.
    auto rowbase = [&](int r) {
        return a.qout ? (int)(2 * (blockIdx.x + (unsigned)(r >> 1) * gridDim.x) + (r & 1)) * 16
                      : (int)(blockIdx.x + (unsigned)r * gridDim.x) * 16;
    };
    // The input runs first (loads return in order), then the first item's
    // weights, all unconditional: tokens, rows, blocks and runs are clamped.
    const int half = wave >> 2, tb = half ? TH : 0, tn = half ? MT - TH : TH;
    const int nr = a.n_in / 16, run0 = tid & 255, run = min(run0, nr - 1);
    const bool mine = run0 < nr;
    float4 xv[TH][4], nw[4];
    const float *nwp = a.norm_w ? a.norm_w : a.xin;
#pragma unroll
    for (int j = 0; j < TH; j++)
#pragma unroll
        for (int q = 0; q < 4; q++)
            xv[j][q] = *(const float4 *)(a.xin + (int64_t)min(tb + j, a.M - 1) * a.xin_stride + 16 * run + 4 * q);
#pragma unroll
    for (int q = 0; q < 4; q++) nw[q] = *(const float4 *)(nwp + 16 * run + 4 * q);
    // The input in (a wait the compiler sees: it then has no load of its own
    // left to wait for, and never waits for the weight requests, which it
    // does not see), then the first item's weights, in flight through the
    // norm and the quantization.
    wait_vmcnt<0>();
    issue(rowbase(0), min(b0, a.nb - 1), 0);
    float sc[TH];
#pragma unroll
    for (int j = 0; j < TH; j++) sc[j] = 1.f;
    if (a.norm_w) {  // engine/src/cpu_backend.cpp:48-53, per token; the 4 waves of a half in order
#pragma unroll
        for (int j = 0; j < TH; j++) {
            float ss = 0.f;
#pragma unroll
            for (int q = 0; q < 4; q++)
                ss += xv[j][q].x * xv[j][q].x + xv[j][q].y * xv[j][q].y + xv[j][q].z * xv[j][q].z +
                      xv[j][q].w * xv[j][q].w;
            ss = wave_sum_dpp(mine ? ss : 0.f);
            if (l == 0 && j < tn) ssr[tb + j][wave & 3] = ss;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < TH; j++) {
            const int t = min(tb + j, MT - 1);
            float ss = 0.f;
#pragma unroll
            for (int w = 0; w < 4; w++) ss += ssr[t][w];
            sc[j] = 1.0f / sqrtf(ss / (float)a.n_in + a.eps);
        }
    }
#pragma unroll
    for (int j = 0; j < TH; j++) {
        float v[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float4 f = xv[j][q], g = nw[q];
            v[4 * q] = f.x, v[4 * q + 1] = f.y, v[4 * q + 2] = f.z, v[4 * q + 3] = f.w;
            if (a.norm_w) {
                v[4 * q] = v[4 * q] * sc[j] * g.x, v[4 * q + 1] = v[4 * q + 1] * sc[j] * g.y;
                v[4 * q + 2] = v[4 * q + 2] * sc[j] * g.z, v[4 * q + 3] = v[4 * q + 3] * sc[j] * g.w;
            }
        }
        // quant_run_m pairs adjacent lanes (runs 2g, 2g + 1): nr is a
        // multiple of 16, so both or neither are `mine`.
        if (j < tn && tb + j < a.M && mine) quant_run_m(v, run, lx + (tb + j) * tstride);
    }
    __syncthreads();
    float acc[RT][NW][NA];
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int m = 0; m < NW; m++)
#pragma unroll
            for (int tt = 0; tt < NA; tt++) acc[r][m][tt] = 0.f;
    // Items (row tile r, block b), the tiles outermost, through the two
    // weight slots in turn (tiles innermost, sharing a block's activation
    // fragments, held too many registers); an item reads its block's
    // activation fragments from LDS. Before an item's request for the next
    // one: the LDS reads of the slot it overwrites are in (lgkmcnt 0); before
    // its fragment reads: its own requests are in. Past the last item the
    // request repeats one, in bounds and unused.
    int sl = 0;
#pragma unroll
    for (int r = 0; r < RT; r++) {
        const bool rin = rowbase(r) + rl < a.nrows;
        for (int b = b0; b < b1; b++) {
            const bool lastb = b + 1 >= b1;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(rowbase(lastb ? min(r + 1, RT - 1) : r), lastb ? b0 : b + 1, sl ^ 1);
            wait_vm_n<3 * NW>();
            MAFrag<FMT, NT, P5> xc;
            load_mafrag_at<FMT, NT, P5>(lx, tstride, a.M, b, l, xc);
            gm_prescale<FMT, NT, P5>(xc, kq);
            MWFrag<FMT, NW> w;
            fetch(sl, w);
            gm_item<FMT, NW, NT, P5, NA>(w, xc, acc[r], rin, kq);
            TS5_GM_SB();  // one item at a time
            sl ^= 1;
        }
    }
    // The waves' sums, [r][m][tt][lane] in each wave's own weight slots once
    // its last (repeated) request is in.
    wait_vm_n<0>();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    static_assert(RT * NA * 64 * sizeof(float) <= 2 * WSLOT, "the waves' sums fit their weight slots");
    auto red = [&](int w) { return (float *)(lx + (size_t)a.M * tstride + (size_t)w * 2 * NW * WSLOT); };
#pragma unroll
    for (int r = 0; r < RT; r++)
#pragma unroll
        for (int m = 0; m < NW; m++)
#pragma unroll
            for (int tt = 0; tt < NA; tt++) red(wave)[((r * NW + m) * NA + tt) * 64 + l] = acc[r][m][tt];
    __syncthreads();
    constexpr int E = RT * NA * 64;  // entries (row tile, token tile, lane)
    static_assert(E <= 64 * GX_WAVES, "one entry a thread");
    float *ys = (float *)(lx + (size_t)a.M * tstride + (size_t)GX_WAVES * 2 * NW * WSLOT);  // qout: [MT][RT * 16]
    if (tid < E) {
        const int r = tid / (NA * 64), tt = (tid / 64) % NA, ln = tid & 63;
        auto wsum = [&](int m, int lane) {
            float v = 0.f;
#pragma unroll
            for (int w = 0; w < GX_WAVES; w++) v += red(w)[((r * NW + m) * NA + tt) * 64 + lane];
            return v;
        };
        float v[NW];
#pragma unroll
        for (int m = 0; m < NW; m++) {
            if (P5 && tt == NT) {  // the fifth token: the four lane groups' shares of the row, (g0 + g1) + (g2 + g3)
                const int lr = ln & 15;
                v[m] = (wsum(m, lr) + wsum(m, lr + 16)) + (wsum(m, lr + 32) + wsum(m, lr + 48));
            } else {
                v[m] = wsum(m, ln);
            }
        }
        const int row = rowbase(r) + (ln & 15), tok = tt == NT ? 4 : 4 * tt + (ln >> 4);
        if (row < a.nrows && tok < a.M && (tt < NT || (ln >> 4) == 0)) {
            const int64_t o = (int64_t)tok * a.ldy + row;
            float y;
            if (MODE == G_ADD) y = a.y_in[o] + v[0];
            else if (MODE == G_GLU) y = glu_act(v[0], v[NW - 1], a.gelu);
            else y = v[0];
            a.out[o] = y;
            if (a.qout) ys[(tok * RT + r) * 16 + (ln & 15)] = y;
        }
    }
    if (a.qout) {
        // Each (token, row tile) as a 16-value run of the next matmul's
        // records: quant_run_m (the pairs of one 32-row chunk in adjacent
        // lanes, RT even), as k_act_quant_m would write them from y.
        static_assert(RT % 2 == 0 || RT == 1, "row tiles in pairs");
        __syncthreads();
        constexpr int MT = P5 ? 5 : 4;
        if (tid < MT * RT) {
            const int tok = tid / RT, run = tid % RT, row0 = rowbase(run);
            if (tok < a.M && row0 < a.nrows) {
                float v[16];
#pragma unroll
                for (int i = 0; i < 16; i++) v[i] = ys[(tok * RT + run) * 16 + i];
                quant_run_m(v, row0 / 16, a.qout + (int64_t)tok * mact_bytes(a.nrows));
            }
        }
    }
}

// ---------------------------------------------------------------------------
// The same small-batch matmul (Q4_K, 1-5 tokens, no gate/up) over activation
// records already in memory (k_act_quant_m's, for inputs wider than the
// fused kernel's LDS holds: the down projection), one workgroup of 8 waves a
// CU walking row tiles gridDim.x apart. Per item (row tile, block of the
// wave's eighth) both the weights (16 rows x 144 bytes) and the block's
// records of the M tokens (M x 896 bytes) come into the wave's LDS slots by
// DMA, one item ahead; the waves' sums of a tile meet in LDS and a thread
// per (token tile, lane) finishes the tile's outputs.
// ---------------------------------------------------------------------------
template <int MODE, int TM>
__global__ __launch_bounds__(64 * GX_WAVES) void k_gemm_mw(GemmArgs a) {
    constexpr int FMT = F_Q4K, NW = 1, NT = 1;
    constexpr bool P5 = TM == 5;
    static_assert(MODE != G_GLU && (TM == 1 || TM == 5), "wide small-batch matmul: up to 5 tokens, one matrix");
    constexpr int NA = NT + (P5 ? 1 : 0);
    constexpr int WSLOT = 16 * Q4K_BYTES, RSLOT = 5 * 1024;  // weights; records (5 requests of 64 x 16 B)
    extern __shared__ __align__(16) uint8_t lw[];  // per wave: 2 weight slots, 2 record slots; then the sums
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l = tid & 63, kq = l >> 4, rl = l & 15;
    const int ntile = (a.nrows + 15) / 16;
    const int bpq = (a.nb + GX_WAVES - 1) / GX_WAVES, b0 = wave * bpq, b1 = min(a.nb, b0 + bpq);
    uint8_t *wst = lw + (size_t)wave * 2 * (WSLOT + RSLOT), *rst = wst + 2 * WSLOT;
    float *red = (float *)(lw + (size_t)GX_WAVES * 2 * (WSLOT + RSLOT));  // [wave][tt][64]
    const uint32_t wbytes = (uint32_t)a.nrows * a.nb * Q4K_BYTES;  // rows past the last read zeros
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(a.w, wbytes);
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(a.act, (uint32_t)(a.M * a.act_stride));
    // Weight pieces: c = 64 i + lane, row c / 9, bytes 16 (c % 9). Record
    // pieces: c = 64 i + lane, token c / 56 (past the M tokens: the last
    // one's, into LDS past the records, unused), bytes 16 (c % 56).
    uint32_t coff[3], roff[5];
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const int c = min(64 * i + l, 143);
        coff[i] = (uint32_t)((c / 9) * a.nb * Q4K_BYTES + 16 * (c % 9));
    }
#pragma unroll
    for (int i = 0; i < 5; i++) {
        const int c = 64 * i + l, t = min(c / 56, a.M - 1);
        roff[i] = (uint32_t)(t * a.act_stride + 16 * (c % 56));
    }
    auto issue = [&](int tile, int b, int slot) {
        uint32_t wb = ((uint32_t)tile * 16 * a.nb + b) * Q4K_BYTES, rb = (uint32_t)b * MACT_BLOCK;
        asm volatile("" : "+s"(wb), "+s"(rb));  // opaque: the per-lane sums are formed here
#pragma unroll
        for (int i = 0; i < 3; i++)
            if (i < 2 || l < 16) dma16b(rw, wb + coff[i], lds_addr(wst + slot * WSLOT + 1024 * i));
#pragma unroll
        for (int i = 0; i < 5; i++) dma16b(ra, rb + roff[i], lds_addr(rst + slot * RSLOT + 1024 * i));
    };
    int sl = 0;
    issue(blockIdx.x, min(b0, a.nb - 1), 0);
    for (int tile = blockIdx.x; tile < ntile; tile += gridDim.x) {
        const bool rin = tile * 16 + rl < a.nrows;
        float acc[NW][NA];
#pragma unroll
        for (int tt = 0; tt < NA; tt++) acc[0][tt] = 0.f;
        for (int b = b0; b < b1; b++) {
            // The next item: the next block, or the next tile's first (past
            // the last tile a repeat, in bounds and unused).
            const bool lastb = b + 1 >= b1;
            const int ntl = lastb ? min(tile + (int)gridDim.x, ntile - 1) : tile;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(ntl, lastb ? b0 : b + 1, sl ^ 1);
            wait_vm_n<8>();  // this item's 8 requests are in
            MAFrag<FMT, NT, P5> xc;
            load_mafrag_at<FMT, NT, P5>(rst + sl * RSLOT, MACT_BLOCK, a.M, 0, l, xc);
            gm_prescale<FMT, NT, P5>(xc, kq);
            MWFrag<FMT, NW> w;
            const uint8_t *p = wst + sl * WSLOT + Q4K_BYTES * rl;
            w.hdr[0] = *(const uint4 *)p;
#pragma unroll
            for (int g = 0; g < 4; g++) w.q[0][g] = *(const uint64_t *)(p + 16 + 32 * g + 8 * kq);
            gm_item<FMT, NW, NT, P5, NA>(w, xc, acc, rin, kq);
            TS5_GM_SB();  // one item at a time
            sl ^= 1;
        }
#pragma unroll
        for (int tt = 0; tt < NA; tt++) red[(wave * NA + tt) * 64 + l] = acc[0][tt];
        __syncthreads();
        if (tid < NA * 64) {
            const int tt = tid / 64, ln = tid & 63;
            auto wsum = [&](int lane) {
                float v = 0.f;
#pragma unroll
                for (int w2 = 0; w2 < GX_WAVES; w2++) v += red[(w2 * NA + tt) * 64 + lane];
                return v;
            };
            float v;
            if (P5 && tt == NT) {  // the fifth token: (g0 + g1) + (g2 + g3)
                const int lr = ln & 15;
                v = (wsum(lr) + wsum(lr + 16)) + (wsum(lr + 32) + wsum(lr + 48));
            } else {
                v = wsum(ln);
            }
            const int row = tile * 16 + (ln & 15), tok = tt == NT ? 4 : 4 * tt + (ln >> 4);
            if (row < a.nrows && tok < a.M && (tt < NT || (ln >> 4) == 0)) {
                const int64_t o = (int64_t)tok * a.ldy + row;
                if (MODE == G_ADD) a.out[o] = a.y_in[o] + v;
                else a.out[o] = v;
            }
        }
        __syncthreads();  // the sums are read before the next tile writes them
    }
    wait_vm_n<0>();  // the last (repeated) requests are in before the waves end
}

// ---------------------------------------------------------------------------
// Q6_K rows for 1-5 tokens over activation records (the verify batch's head,
// 128256 x 4096): one workgroup of 8 waves a CU holds the M tokens' records
// of all nb blocks in LDS; each wave takes whole 16-row tiles (tile
// blockIdx.x * 8 + wave, then every 8 gridDim.x-th), item by item over the
// blocks, each item's 16 rows x 208 bytes and their 16 f16 scales brought
// into the wave's LDS slot by DMA one item ahead; no cross-wave sums.
// ---------------------------------------------------------------------------
__device__ inline void dma4b(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t lds_base) {
    asm volatile("buffer_load_dword %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds_base) : "memory");
}
constexpr int MH_SLOT = 16 * Q6K_BODY + 64;  // 16 rows' bodies, then their scales (a dword each)
static size_t gemm_mh_lds(int M, int nb) { return (size_t)M * nb * MACT_BLOCK + (size_t)GX_WAVES * 2 * MH_SLOT; }

template <int TM>
__global__ __launch_bounds__(64 * GX_WAVES) void k_gemm_mh(GemmArgs a) {
    constexpr int FMT = F_Q6K, NW = 1, NT = 1;
    constexpr bool P5 = TM == 5;
    static_assert(TM == 1 || TM == 5, "small-batch head: up to 5 tokens");
    constexpr int NA = NT + (P5 ? 1 : 0);
    extern __shared__ __align__(16) uint8_t lh[];  // the records [M][nb][896], then each wave's 2 slots
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l = tid & 63, kq = l >> 4, rl = l & 15;
    const int nb = a.nb, ntile = (a.nrows + 15) / 16;
    const int rstride = nb * MACT_BLOCK;  // a token's records in LDS
    uint8_t *rec = lh, *wst = lh + (size_t)a.M * rstride + (size_t)wave * 2 * MH_SLOT;
    const int64_t nblocks = (int64_t)a.nrows * nb;
    const __amdgpu_buffer_rsrc_t rw = buf_rsrc(a.w, (uint32_t)(nblocks * Q6K_BODY));  // past the last row: zeros
    const __amdgpu_buffer_rsrc_t rs = buf_rsrc(a.s, (uint32_t)(nblocks * 2));
    const __amdgpu_buffer_rsrc_t ra = buf_rsrc(a.act, (uint32_t)(a.M * a.act_stride));
    // Weight pieces: c = 64 i + lane (the fourth request: lanes 0-15), row
    // c / 13, bytes 16 (c % 13); lanes 0-15 also bring row lane's scale (the
    // aligned dword that holds it).
    uint32_t coff[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int c = min(64 * i + l, 207);
        coff[i] = (uint32_t)((c / 13) * nb * Q6K_BODY + 16 * (c % 13));
    }
    auto issue = [&](int tile, int b, int slot) {
        uint32_t wb = ((uint32_t)tile * 16 * nb + b) * Q6K_BODY, sb = (uint32_t)tile * 16 * nb + b;
        asm volatile("" : "+s"(wb), "+s"(sb));  // opaque: the per-lane sums are formed here
        uint8_t *dst = wst + slot * MH_SLOT;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (i < 3 || l < 16) dma16b(rw, wb + coff[i], lds_addr(dst + 1024 * i));
        if (l < 16) dma4b(rs, ((sb + (uint32_t)l * nb) * 2) & ~3u, lds_addr(dst + 16 * Q6K_BODY));
    };
    // The records (pieces p of M * nb * 56, 16 bytes each, in order), then
    // the first item; all in before any wave reads the records.
    const int npieces = a.M * nb * (MACT_BLOCK / 16), tpc = nb * (MACT_BLOCK / 16);
    for (int k = 0; 64 * GX_WAVES * k < npieces; k++) {
        const int p = 64 * GX_WAVES * k + tid;
        if (p < npieces)
            dma16b(ra, (uint32_t)((p / tpc) * a.act_stride + 16 * (p % tpc)),
                   lds_addr(rec + 16 * (64 * GX_WAVES * k + 64 * wave)));
    }
    const int gw = blockIdx.x * GX_WAVES + wave, nwv = gridDim.x * GX_WAVES;
    issue(min(gw, ntile - 1), 0, 0);
    wait_vm_n<0>();
    __syncthreads();
    int sl = 0;
    for (int tile = gw; tile < ntile; tile += nwv) {
        const bool rin = tile * 16 + rl < a.nrows;
        float acc[NW][NA];
#pragma unroll
        for (int tt = 0; tt < NA; tt++) acc[0][tt] = 0.f;
        for (int b = 0; b < nb; b++) {
            // The next item: the next block, or the next tile's first (past
            // the wave's last tile a repeat, in bounds and unused).
            const bool lastb = b + 1 >= nb;
            const int ntl = lastb ? min(tile + nwv, ntile - 1) : tile;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue(ntl, lastb ? 0 : b + 1, sl ^ 1);
            wait_vm_n<5>();  // this item's 5 requests are in
            MAFrag<FMT, NT, P5> xc;
            load_mafrag_at<FMT, NT, P5>(rec, rstride, a.M, b, l, xc);
            gm_prescale<FMT, NT, P5>(xc, kq);
            MWFrag<FMT, NW> w;
            const uint8_t *src = wst + sl * MH_SLOT;
            const uint8_t *body = src + Q6K_BODY * rl;
#pragma unroll
            for (int h = 0; h < 2; h++) {
                w.ql[0][h][0] = *(const uint64_t *)(body + 64 * h + 8 * kq);
                w.ql[0][h][1] = *(const uint64_t *)(body + 64 * h + 32 + 8 * kq);
                w.qh[0][h] = *(const uint64_t *)(body + 128 + 32 * h + 8 * kq);
            }
            w.sc[0] = *(const uint4 *)(body + 192);
            const uint32_t dw = *(const uint32_t *)(src + 16 * Q6K_BODY + 4 * rl);
            const uint32_t idx = (uint32_t)(tile * 16 + rl) * nb + b;
            w.d[0] = h2f((dw >> (16 * (idx & 1))) & 0xffff);
            gm_item<FMT, NW, NT, P5, NA>(w, xc, acc, rin, kq);
            TS5_GM_SB();  // one item at a time
            sl ^= 1;
        }
        // Row tile * 16 + lane % 16; token 4 tt + lane / 16, and with P5 the
        // fifth token's four lane groups added ((g0 + g1) + (g2 + g3)).
#pragma unroll
        for (int tt = 0; tt < NA; tt++) {
            float v = acc[0][tt];
            if (P5 && tt == NT) v = add_xor32(add_xor16(v));
            const int row = tile * 16 + rl, tok = tt == NT ? 4 : 4 * tt + kq;
            if (row < a.nrows && tok < a.M && (tt < NT || kq == 0)) a.out[(int64_t)tok * a.ldy + row] = v;
        }
    }
    wait_vm_n<0>();  // the last (repeated) requests are in before the waves end
}

template <int MODE, int TM>
static void launch_gemm_mx_tm(const GemmArgs &a, int rt, unsigned grid, size_t lds, hipStream_t s) {
    if (rt == 4) hipLaunchKernelGGL((k_gemm_mx<MODE, TM, 4>), dim3(grid), dim3(64 * GX_WAVES), lds, s, a);
    else if (rt == 2) hipLaunchKernelGGL((k_gemm_mx<MODE, TM, 2>), dim3(grid), dim3(64 * GX_WAVES), lds, s, a);
    else hipLaunchKernelGGL((k_gemm_mx<MODE, TM, 1>), dim3(grid), dim3(64 * GX_WAVES), lds, s, a);
}

template <int MODE, int TM>
static void launch_gemm_fused_tm(const GemmArgs &a, int rt, size_t lds, hipStream_t s) {
    const unsigned grid = (unsigned)((a.nrows + 16 * rt - 1) / (16 * rt));
    if (rt == 4) hipLaunchKernelGGL((k_gemm_m<F_Q4K, MODE, TM, 4, true>), dim3(grid), dim3(256), lds, s, a);
    else if (rt == 2) hipLaunchKernelGGL((k_gemm_m<F_Q4K, MODE, TM, 2, true>), dim3(grid), dim3(256), lds, s, a);
    else hipLaunchKernelGGL((k_gemm_m<F_Q4K, MODE, TM, 1, true>), dim3(grid), dim3(256), lds, s, a);
}

bool gemm_fused_fits(uint32_t t, int64_t ne0, int M) {
    return t == T_Q4_K && ne0 % 256 == 0 && ne0 <= 4096 && M >= 1 && M <= 5;
}

bool gemm_fused_qout_fits(int64_t ne0, int64_t ne1, int M) {
    const int64_t pairs = (ne1 + 31) / 32, grid = std::min<int64_t>(pairs, g_gemm_m_cu);
    return gemm_fused_fits(T_Q4_K, ne0, M) && ne1 % 256 == 0 && (pairs + grid - 1) / grid <= 2;
}

hipError_t launch_gemm_fused(const void *w, const void *w2, int64_t ne0, int64_t ne1, const float *x,
                             int64_t xstride, const float *norm_w, float eps, int M, int mode, float *y,
                             const float *y_in, int64_t ldy, hipStream_t s, void *qout) {
    if (!gemm_fused_fits(T_Q4_K, ne0, M)) return hipErrorInvalidValue;
    if (qout && !gemm_fused_qout_fits(ne0, ne1, M)) return hipErrorInvalidValue;
    GemmArgs a{};
    a.gelu = (mode & GLU_GELU) ? 1 : 0;
    mode &= ~GLU_GELU;
    a.t = T_Q4_K, a.w = (const uint8_t *)w, a.w2 = (const uint8_t *)w2, a.nrows = (int)ne1;
    a.nb = (int)(ne0 / 256), a.n_in = (int)ne0, a.M = M, a.ks = 1, a.out = y, a.y_in = y_in, a.ldy = ldy;
    a.xin = x, a.xin_stride = xstride, a.norm_w = norm_w, a.eps = eps, a.qout = (uint8_t *)qout;
    const size_t lds = (size_t)M * a.nb * MACT_BLOCK;
    const int tiles = (a.nrows + 15) / 16;
    // qout: tiles in pairs, pairs gridDim.x apart (2 or 4 tiles a workgroup).
    const int units = qout ? (tiles + 1) / 2 : tiles;
    const unsigned grid = (unsigned)std::min(units, g_gemm_m_cu);
    const int rt_mx = (qout ? 2 : 1) * ((units + (int)grid - 1) / (int)grid);
    if (rt_mx <= 4) {
        // One workgroup a CU (at most), each RT tiles gridDim.x apart; its
        // LDS: the records, then each wave's two weight slots of 16 rows x
        // 144 B per matrix (GLU: 72 KiB; with the records' 5 x 16 x 896 B
        // under 160 KiB), then (qout) the outputs of its tiles.
        const int rtp = rt_mx > 2 ? 4 : rt_mx;
        const int nw = mode == G_GLU ? 2 : 1;
        const size_t lds_mx = lds + (size_t)GX_WAVES * 2 * nw * 16 * Q4K_BYTES + (qout ? 5 * 4 * 16 * sizeof(float) : 0);
        auto go = [&](auto mode_c) {
            constexpr int MD = decltype(mode_c)::value;
            if (M == 5) launch_gemm_mx_tm<MD, 5>(a, rtp, grid, lds_mx, s);
            else launch_gemm_mx_tm<MD, 1>(a, rtp, grid, lds_mx, s);
        };
        if (mode == G_ADD) go(std::integral_constant<int, G_ADD>{});
        else if (mode == G_GLU) go(std::integral_constant<int, G_GLU>{});
        else go(std::integral_constant<int, G_STORE>{});
        return hipGetLastError();
    }
    int rt = tiles >= 4 * g_gemm_m_cu ? 4 : tiles >= 2 * g_gemm_m_cu ? 2 : 1;
    if (GM_RTMAX < rt) rt = GM_RTMAX;
    auto go = [&](auto mode_c) {
        constexpr int MD = decltype(mode_c)::value;
        if (M == 5) launch_gemm_fused_tm<MD, 5>(a, rt, lds, s);
        else launch_gemm_fused_tm<MD, 1>(a, rt, lds, s);
    };
    if (mode == G_ADD) go(std::integral_constant<int, G_ADD>{});
    else if (mode == G_GLU) go(std::integral_constant<int, G_GLU>{});
    else go(std::integral_constant<int, G_STORE>{});
    return hipGetLastError();
}

// Q4_K: 1-8 tokens; Q6_K (not the fused gate/up): 1-5 tokens.
template <int FMT, int MODE>
static bool gemm_m_fits(int M) {
    if constexpr (FMT == F_Q4K) return M <= 8;
    else if constexpr (FMT == F_Q6K && MODE != G_GLU) return M <= 5;
    else return false;
}

template <int FMT, int MODE>
static hipError_t launch_gemm_m(const GemmArgs &a, hipStream_t s) {
    // Row tiles a workgroup: as many as keep about one workgroup a CU.
    const int tiles = (a.nrows + 15) / 16;
    int rt = tiles >= 4 * g_gemm_m_cu ? 4 : tiles >= 2 * g_gemm_m_cu ? 2 : 1;
    if (GM_RTMAX < rt) rt = GM_RTMAX;
    if (a.M <= 4) launch_gemm_m_nt<FMT, MODE, 1>(a, rt, s);
    else if (a.M == 5) launch_gemm_m_nt<FMT, MODE, 5>(a, rt, s);
    else if constexpr (FMT == F_Q4K) launch_gemm_m_nt<FMT, MODE, 2>(a, rt, s);
    return hipGetLastError();
}

// Split-K: y[t][r] = (y_in +) sum over splits in order (GLU: act(g) * u).
// Four consecutive values a thread (rows of one token when nrows % 4 == 0,
// else one value at a time), every split's partial requested before the
// first is added; the sums run in split order.
template <int MODE>
__device__ inline void gemm_reduce_one(const float *__restrict__ part, int ks, int64_t n, int nrows, int64_t e,
                                       float *y, const float *y_in, int64_t ldy, int gelu) {
    float g = 0.f, u = 0.f;
    for (int k = 0; k < ks; k++) {
        g += part[(int64_t)k * 2 * n + e];
        if (MODE == G_GLU) u += part[(int64_t)k * 2 * n + n + e];
    }
    const int tok = (int)(e / nrows), r = (int)(e % nrows);
    const int64_t o = (int64_t)tok * ldy + r;
    if (MODE == G_ADD) y[o] = y_in[o] + g;
    else if (MODE == G_GLU) y[o] = glu_act(g, u, gelu);
    else y[o] = g;
}

template <int MODE>
__global__ __launch_bounds__(256) void k_gemm_reduce(const float *__restrict__ part, int ks, int M, int nrows, float *y,
                                                     const float *y_in, int64_t ldy, int gelu) {
    const int64_t n = (int64_t)M * nrows;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    if (nrows % 4) {
        for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < n; e += stride)
            gemm_reduce_one<MODE>(part, ks, n, nrows, e, y, y_in, ldy, gelu);
        return;
    }
    constexpr int KC = 8;  // splits requested at once
    for (int64_t e = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x); e < n; e += 4 * stride) {
        float4 g = make_float4(0.f, 0.f, 0.f, 0.f), u = g;
        for (int k0 = 0; k0 < ks; k0 += KC) {
            float4 pg[KC], pu[KC];
#pragma unroll
            for (int k = 0; k < KC; k++) {
                if (k0 + k < ks) {
                    pg[k] = *(const float4 *)(part + (int64_t)(k0 + k) * 2 * n + e);
                    if (MODE == G_GLU) pu[k] = *(const float4 *)(part + (int64_t)(k0 + k) * 2 * n + n + e);
                }
            }
#pragma unroll
            for (int k = 0; k < KC; k++) {
                if (k0 + k < ks) {
                    g.x += pg[k].x, g.y += pg[k].y, g.z += pg[k].z, g.w += pg[k].w;
                    if (MODE == G_GLU) u.x += pu[k].x, u.y += pu[k].y, u.z += pu[k].z, u.w += pu[k].w;
                }
            }
        }
        const int tok = (int)(e / nrows), r = (int)(e % nrows);
        float *o = y + (int64_t)tok * ldy + r;
        const float gv[4] = {g.x, g.y, g.z, g.w}, uv[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (MODE == G_ADD) o[j] = y_in[(int64_t)tok * ldy + r + j] + gv[j];
            else if (MODE == G_GLU) o[j] = glu_act(gv[j], uv[j], gelu);
            else o[j] = gv[j];
        }
    }
}

static hipError_t launch_gemm_reduce(const float *part, int ks, int M, int nrows, int mode, float *y, const float *y_in,
                                     int64_t ldy, int gelu, hipStream_t s) {
    const int64_t n = (int64_t)M * nrows, per = nrows % 4 ? 1 : 4;
    const dim3 g((unsigned)std::min<int64_t>(4096, (n / per + 255) / 256)), b(256);
    if (mode == G_ADD) hipLaunchKernelGGL(k_gemm_reduce<G_ADD>, g, b, 0, s, part, ks, M, nrows, y, y_in, ldy, 0);
    else if (mode == G_GLU) hipLaunchKernelGGL(k_gemm_reduce<G_GLU>, g, b, 0, s, part, ks, M, nrows, y, y_in, ldy, gelu);
    else hipLaunchKernelGGL(k_gemm_reduce<G_STORE>, g, b, 0, s, part, ks, M, nrows, y, y_in, ldy, 0);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Past 16 tokens Q4_K rows take the fp16 prompt matmul (launch_gemm_wide), so
// k_gemm is built for Q6_K and Q8_0 only.
template <int FMT, int MODE>
static hipError_t gemm_go(const GemmArgs &a, dim3 grid, int tn, hipStream_t s) {
    if constexpr (FMT == F_Q4K || (FMT == F_Q6K && MODE != G_GLU)) {
        // Q4_K up to 8 tokens and Q6_K up to 5 (the verify batch's head) on
        // k_gemm_m; the rest on k_gemm_small.
        if constexpr (FMT == F_Q4K && MODE != G_GLU)
            if (a.M <= 5 && a.ks == 1) {
                const int tiles = (a.nrows + 15) / 16;
                const size_t lds = (size_t)GX_WAVES * 2 * (16 * Q4K_BYTES + 5 * 1024) + GX_WAVES * 2 * 64 * 4;
                const dim3 g((unsigned)std::min(tiles, g_gemm_m_cu)), blk(64 * GX_WAVES);
                if (a.M == 5) hipLaunchKernelGGL((k_gemm_mw<MODE, 5>), g, blk, lds, s, a);
                else hipLaunchKernelGGL((k_gemm_mw<MODE, 1>), g, blk, lds, s, a);
                return hipGetLastError();
            }
        if constexpr (FMT == F_Q6K && MODE == G_STORE)
            if (a.M <= 5 && a.ks == 1 && gemm_mh_lds(a.M, a.nb) <= 160 * 1024) {
                const int tiles = (a.nrows + 15) / 16;
                const dim3 g((unsigned)std::min((tiles + GX_WAVES - 1) / GX_WAVES, g_gemm_m_cu)), blk(64 * GX_WAVES);
                const size_t lds = gemm_mh_lds(a.M, a.nb);
                if (a.M == 5) hipLaunchKernelGGL((k_gemm_mh<5>), g, blk, lds, s, a);
                else hipLaunchKernelGGL((k_gemm_mh<1>), g, blk, lds, s, a);
                return hipGetLastError();
            }
        if (gemm_m_fits<FMT, MODE>(a.M)) return launch_gemm_m<FMT, MODE>(a, s);
    }
    if (a.M <= 16) {
        hipLaunchKernelGGL((k_gemm_small<FMT, MODE>), dim3((a.nrows + 15) / 16), dim3(256), 0, s, a);
    } else if constexpr (q8_rows<FMT>) {
        if (tn == 4) hipLaunchKernelGGL((k_gemm<FMT, MODE, 4>), grid, dim3(256), 0, s, a);
        else hipLaunchKernelGGL((k_gemm<FMT, MODE, 1>), grid, dim3(256), 0, s, a);
    } else if constexpr (FMT == F_Q6K) {
        hipLaunchKernelGGL((k_gemm<FMT, MODE, 1>), grid, dim3(256), 0, s, a);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int MODE>
static hipError_t gemm_fmt(const GemmArgs &a, dim3 grid, int tn, hipStream_t s) {
    switch (a.t) {
    case T_Q4_K: return gemm_go<F_Q4K, MODE>(a, grid, tn, s);
    case T_Q6_K: return gemm_go<F_Q6K, MODE>(a, grid, tn, s);
    case T_Q8_0: return gemm_go<F_Q80, MODE>(a, grid, tn, s);
    case T_Q8SM: return gemm_go<F_Q8M, MODE>(a, grid, tn, s);
    }
    return hipErrorInvalidValue;
}

// Token groups of 16 per wave: 4 for Q8_0 batches past 16 tokens (Q6_K rows
// keep 1: its 4-group kernel does not fit the register file).
static int gemm_tn(uint32_t t, int M) { return M > 16 && (t == T_Q8_0 || t == T_Q8SM) ? 4 : 1; }

static int g_gemm_cu = 256;
void set_gemm_cu_count(int n) { g_gemm_cu = g_gemm_m_cu = n > 0 ? n : 256; }

// Splits of K that give the launch about four workgroups per CU when the
// tokens alone do not (small M: the matmul is a weight stream).
static int gemm_splits(int64_t rows, int M, int nb, int tn) {
    if (M <= 16) return 1;  // k_gemm_small splits the blocks inside the workgroup
    const int64_t wgs = ((rows + 63) / 64) * ((M + 16 * tn - 1) / (16 * tn));
    int ks = (int)std::min<int64_t>(16, std::max<int64_t>(1, (4 * g_gemm_cu + wgs - 1) / wgs));
    return std::min(ks, nb);
}

int gemm_act_form(uint32_t t, int64_t n, int ntok) {
    if (n % 256) return GA_ACT;
    if (t == T_Q4_K) return ntok > 16 ? GA_HACT : GA_MACT;
    return t == T_Q6_K ? GA_MACT : GA_ACT;
}

size_t gemm_scratch_bytes(int64_t rows, int M, int nb) {  // the bound for every type
    const int ks = std::max(gemm_splits(rows, M, nb, M > 16 ? 4 : 1), M > 16 ? wide_splits(rows, M, nb, g_gemm_cu, G_ADD) : 1);
    return ks > 1 ? (size_t)ks * 2 * M * rows * 4 : 0;
}

hipError_t launch_gemm(uint32_t t, const void *w, const void *w2, int64_t ne0, int64_t ne1, const void *act, int M,
                       int mode, float *y, const float *y_in, int64_t ldy, void *scratch, hipStream_t s) {
    const int gelu = (mode & GLU_GELU) ? 1 : 0;
    mode &= ~GLU_GELU;
    GemmArgs a{};
    a.gelu = gelu;
    a.t = t, a.w = (const uint8_t *)w, a.w2 = (const uint8_t *)w2, a.nrows = (int)ne1;
    a.nb = (int)(ne0 / block_values(t)), a.n_in = (int)ne0, a.M = M, a.act = (const uint8_t *)act;
    if (gemm_act_form(t, ne0, M) == GA_HACT) {
        const int ks = wide_splits(ne1, M, (int)(ne0 / 256), g_gemm_cu, mode);
        hipError_t e = launch_gemm_wide(w, w2, ne0, ne1, act, M, mode | (gelu ? GLU_GELU : 0), y, y_in, ldy, scratch, ks, s);
        if (e != hipSuccess || ks == 1) return e;
        return launch_gemm_reduce((const float *)scratch, ks, M, (int)ne1, mode, y, y_in, ldy, gelu, s);
    }
    a.act_stride = (int64_t)gemm_act_bytes(t, ne0, M), a.y_in = y_in, a.ldy = ldy;
    if (split_layout(t)) {  // Q8SM: (scale, min) pairs behind the quants, read as float2
        const int64_t nblocks = (int64_t)a.nb * ne1;
        a.s = (const uint16_t *)(a.w + split_scale_offset(t, nblocks));
        a.s2 = w2 ? (const uint16_t *)(a.w2 + split_scale_offset(t, nblocks)) : nullptr;
    }
    const int tn = gemm_tn(t, M);
    a.ks = gemm_splits(ne1, M, a.nb, tn);
    a.out = a.ks > 1 ? (float *)scratch : y;
    const dim3 grid((unsigned)((ne1 + 63) / 64), (unsigned)((M + 16 * tn - 1) / (16 * tn)), (unsigned)a.ks);
    hipError_t e = mode == G_ADD ? gemm_fmt<G_ADD>(a, grid, tn, s)
                   : mode == G_GLU ? gemm_fmt<G_GLU>(a, grid, tn, s)
                                   : gemm_fmt<G_STORE>(a, grid, tn, s);
    if (e != hipSuccess || a.ks == 1) return e;
    return launch_gemm_reduce((const float *)scratch, a.ks, M, (int)ne1, mode, y, y_in, ldy, gelu, s);
}

}  // namespace ts5hip
