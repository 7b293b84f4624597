// The prompt matmul for Q4_K rows: Y[t] = W x_t for batches past 16 tokens
// (the reference's matmul_big path for prompts, engine/src/vk_backend.cpp:
// 866-918; its CPU restatement engine/src/cpu_backend.cpp:18-41).
//
// fp16 matrix cores with exact operands. A Q4_K weight is d*sc_s*q - dmin*m_s
// (q 0..15, sc_s and m_s 6-bit per 32-value sub-block s; quants.cpp:133-160),
// so per 256-value block
//   y += d * sum_s sum_k (sc_s q_k) x_k  -  dmin * sum_s m_s X_s
// with X_s the sub-block's sum of x. Both inner sums run on the matrix cores:
//  * sc_s q <= 945 is an exact fp16 integer, so the A operand carries the
//    sub-block scale and one fp32 accumulator P collects all 8 sub-blocks of a
//    block (16 v_mfma_f32_16x16x32_f16 per 16x16 tile and block);
//  * the activations arrive as two fp16 planes of x 2^-e (hi + lo, about 22
//    bits; the per-token power of two keeps the residual stream's 1e11-sized
//    values in range), each multiplied into P by its own MFMA;
//  * the min term is one v_mfma_f32_16x16x16_f16 per tile and block: lane
//    group k (of 4) carries (m_2k, m_2k+1, m_2k, m_2k+1) against the hi and lo
//    halves of (X_2k, X_2k+1) / 32.
// Per block and output only y += d P - 32 dmin Q is left for the VALU, and
// y = acc 2^e at the end.
//
// Workgroup: 4 waves x (2 row tiles of 16) x 128 tokens (8 token tiles): GLU
// waves take 16 rows of gate and the same 16 of up, the others 32 rows. The K
// loop runs in stages of a quarter block (64 values, two sub-blocks), two
// stages in LDS: the one computed and the next, brought in by DMA
// (global_load_lds_*, from an SGPR or per-lane base and fixed per-lane
// offsets) while the current one is computed. The loop issues no register
// loads, so the only waits are the explicit vmcnt ones. A token's 16 pieces of
// 16 bytes per stage sit at piece ^ (token & 15), so the 16 lanes that read
// one piece of 16 tokens hit 16 different bank groups. Split-K (grid z, whole
// blocks) when rows x tokens alone give too few workgroups; a second kernel
// adds the partial sums in a fixed order.
//
// Lane layout of the 16x16x32 MFMA: A lane l = row l%16, k-group l/16 (8
// values); B lane l = token l%16, the same k-group; D lane l = rows
// 4*(l/16)+i of token l%16 (16x16x16: 4 values per k-group, the same D). The
// k order inside an MFMA only has to agree between A and B.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace ts5hip {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

struct WideArgs {
    const uint8_t *w, *w2;  // Q4_K rows (w2: GLU's up projection)
    const uint8_t *act;     // M records of hact_bytes(n_in)
    int64_t act_stride;
    float *out;             // ks == 1: y [M][ldy]; ks > 1: partials [ks][2][M][nrows]
    const float *y_in;      // W_ADD: residual [M][ldy] (may be out)
    int64_t ldy;
    int nrows, nb, n_in, M, ks;
    int gelu;  // W_GLU: GELU (tanh form) for SiLU
};

enum { W_STORE = 0, W_ADD = 1, W_GLU = 2 };
constexpr int WG_TOK = 128;
__host__ __device__ constexpr int wide_rows(int mode) { return mode == W_GLU ? 64 : 128; }

// LDS: two stages of 39 KB (two workgroups per CU).
struct WideStage {
    uint4 b[WG_TOK * 16];  // [token][piece ^ (token & 15)]: hi pieces 0..7, lo 8..15
    uint2 x[WG_TOK];       // [token]: (hi_0, hi_1), (lo_0, lo_1) of the quarter's sums / 32
    uint4 wq[4][32][2];    // [wave][pair * 16 + row]: the 32 quant bytes of sub-blocks 2 q4, 2 q4 + 1
    uint4 wh[4][32];       // [wave][pair * 16 + row]: block header (d, dmin, scales)
};

__device__ inline void dma16s(const uint8_t *sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_base) : "memory");
}
__device__ inline void dma4s(const uint8_t *sbase, uint32_t voff, uint32_t lds_base) {
    asm volatile("global_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "{m0}"(lds_base) : "memory");
}

// Per-lane DMA sources of a workgroup (constant over the K loop but for the
// block offset).
struct WideLanes {
    uint32_t act[8];     // activation pieces 64 (8 wave + i) + lane: token and piece offsets
    uint32_t xs;         // quarter sums: token 32 wave + lane / 2, dword lane & 1
    const uint8_t *q;    // quants: (pair, row) = (lane / 32, lane / 2 % 16), half lane & 1 (block 0)
    const uint8_t *hdr;  // headers: (pair, row) = (lane / 16, lane % 16), lanes < 32 (block 0)
};

// Stage (block b, quarter Q4) into LDS stage S.
template <int Q4>
__device__ inline void wide_issue(const WideArgs &a, WideStage &S, int b, int wave, int lane, const WideLanes &o,
                                  const uint8_t *act_base) {
    const uint8_t *ab = act_base + (int64_t)b * 1024 + Q4 * 128;
#pragma unroll
    for (int i = 0; i < 8; i++) dma16s(ab, o.act[i], lds_addr(S.b) + 1024 * (8 * wave + i));
    dma4s(act_base + hact_x(a.n_in) + (int64_t)(4 * b + Q4) * 8, o.xs, lds_addr(&S.x[32 * wave]));
    dma16(o.q + (int64_t)b * Q4K_BYTES + 32 * Q4, lds_addr(&S.wq[wave][0][0]));
    if (lane < 32) dma16(o.hdr + (int64_t)b * Q4K_BYTES, lds_addr(&S.wh[wave][0]));
}

// 8 quants (one nibble of each of 8 bytes) times the sub-block scale, as
// exact fp16 integers (q sc <= 945): byte -> 0x64bb is 1024 + q, and
// fma(1024 + q, sc, -1024 sc) rounds once, to the exact q sc.
__device__ inline v8h nib_f16(uint2 q, int hi, v2h sc, v2h off) {
    const uint32_t v0 = (hi ? q.x >> 4 : q.x) & 0x0F0F0F0Fu, v1 = (hi ? q.y >> 4 : q.y) & 0x0F0F0F0Fu;
    auto pair = [&](uint32_t v, uint32_t sel) {
        return __builtin_elementwise_fma(__builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, v, sel)), sc, off);
    };
    const v2h p0 = pair(v0, 0x04010400u), p1 = pair(v0, 0x04030402u), p2 = pair(v1, 0x04010400u),
              p3 = pair(v1, 0x04030402u);
    return v8h{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

__device__ inline v2h h2pair(int v) { return v2h{(_Float16)(float)v, (_Float16)(float)v}; }

struct WideAcc {
    float acc[2][8][4];  // [pair][token tile][row i]
    v4f P[2][8];         // the block's sum of sc q x
    v4h xs[8];           // the lane group's quarter sums (hi_0, hi_1, lo_0, lo_1), per token tile
    v4h amin[2];         // the lane group's mins (m_2k, m_2k+1, m_2k, m_2k+1), per pair
};

// One quarter block: Q4 static (its sub-blocks, its lane group for the min
// term, whether it opens or closes the block).
template <int Q4>
__device__ inline void wide_stage(const WideStage &S, WideAcc &R, int wave, int kq, int rl) {
    v2h sc[2][2], off[2][2];
#pragma unroll
    for (int p = 0; p < 2; p++) {
        const uint4 h = S.wh[wave][16 * p + rl];  // the lane's own row
        int sc0, m0, sc1, m1;
        kq_scale_min_pair(Q4, h.y, h.z, h.w, sc0, m0, sc1, m1);
        sc[p][0] = h2pair(sc0), off[p][0] = h2pair(-1024 * sc0);
        sc[p][1] = h2pair(sc1), off[p][1] = h2pair(-1024 * sc1);
        if (kq == Q4) {
            const _Float16 f0 = (_Float16)(float)m0, f1 = (_Float16)(float)m1;
            R.amin[p] = v4h{f0, f1, f0, f1};
        }
    }
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const uint2 xv = S.x[16 * g + rl];
        if (kq == Q4) R.xs[g] = __builtin_bit_cast(v4h, xv);
    }
    uint2 q[2];
#pragma unroll
    for (int p = 0; p < 2; p++) q[p] = *(const uint2 *)((const uint8_t *)&S.wq[wave][16 * p + rl][0] + 8 * kq);
#pragma unroll
    for (int c = 0; c < 2; c++) {
        v8h A[2];
#pragma unroll
        for (int p = 0; p < 2; p++) A[p] = nib_f16(q[p], c, sc[p][c], off[p][c]);
#pragma unroll
        for (int g = 0; g < 8; g++) {
            const int tok = 16 * g + rl;
            const v8h bh = __builtin_bit_cast(v8h, S.b[16 * tok + ((4 * c + kq) ^ rl)]);
            const v8h bl = __builtin_bit_cast(v8h, S.b[16 * tok + ((8 + 4 * c + kq) ^ rl)]);
#pragma unroll
            for (int p = 0; p < 2; p++) {
                const v4f c0 = (Q4 == 0 && c == 0) ? v4f{0.f, 0.f, 0.f, 0.f} : R.P[p][g];
                R.P[p][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[p], bh, c0, 0, 0, 0);
                R.P[p][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[p], bl, R.P[p][g], 0, 0, 0);
            }
        }
    }
    if constexpr (Q4 == 3) {  // block end: acc += d P - 32 dmin sum(m X / 32)
#pragma unroll
        for (int p = 0; p < 2; p++) {
            float d[4], dmin[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t hx = S.wh[wave][16 * p + 4 * kq + i].x;
                d[i] = h2f(hx & 0xffff), dmin[i] = 32.0f * h2f(hx >> 16);
            }
#pragma unroll
            for (int g = 0; g < 8; g++) {
                const v4f Q = __builtin_amdgcn_mfma_f32_16x16x16f16(R.amin[p], R.xs[g], v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; i++)
                    R.acc[p][g][i] = fmaf(d[i], R.P[p][g][i], fmaf(-dmin[i], Q[i], R.acc[p][g][i]));
            }
        }
    }
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void k_gemm_wide(WideArgs a) {
    constexpr int RT = MODE == W_GLU ? 1 : 2;  // row tiles per matrix and wave
    constexpr int ROWS = wide_rows(MODE);
    __shared__ WideStage st[2];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, kq = lane >> 4, rl = lane & 15;
    const int t0 = blockIdx.x * WG_TOK, rw = blockIdx.y * ROWS + 16 * RT * wave;
    const int bps = (a.nb + a.ks - 1) / a.ks, bk0 = blockIdx.z * bps;
    const int nblk = max(0, min(a.nb, bk0 + bps) - bk0);

    WideLanes o;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int u = 64 * (8 * wave + i) + lane, tok = u >> 4, p = (u & 15) ^ (tok & 15);
        o.act[i] = (uint32_t)((min(t0 + tok, a.M - 1) - t0) * a.act_stride) + (p >> 3) * 512 + (p & 7) * 16;
    }
    o.xs = (uint32_t)((min(t0 + 32 * wave + (lane >> 1), a.M - 1) - t0) * a.act_stride) + 4 * (lane & 1);
    auto row_base = [&](int pair, int row) {  // block 0 of the pair's row (clamped)
        const int m = MODE == W_GLU ? pair : 0, rt = MODE == W_GLU ? 0 : pair;
        return (m ? a.w2 : a.w) + (int64_t)min(rw + 16 * rt + row, a.nrows - 1) * a.nb * Q4K_BYTES;
    };
    o.q = row_base(lane >> 5, (lane >> 1) & 15) + 16 + 16 * (lane & 1);
    o.hdr = row_base((lane >> 4) & 1, rl);
    const uint8_t *act_base = a.act + (int64_t)t0 * a.act_stride;

    WideAcc R;
#pragma unroll
    for (int p = 0; p < 2; p++)
#pragma unroll
        for (int g = 0; g < 8; g++)
#pragma unroll
            for (int i = 0; i < 4; i++) R.acc[p][g][i] = 0.f;

    if (nblk > 0) wide_issue<0>(a, st[0], bk0, wave, lane, o, act_base);
    for (int bi = 0; bi < nblk; bi++) {
        const int b = bk0 + bi;
        // Quarter q4 sits in st[q4 & 1]. Each wave waits for its own DMA (the
        // only one in flight); the barrier then makes every wave's DMA visible
        // and frees the other buffer, into which the next quarter goes.
        wait_vm_n<0>();
        __syncthreads();
        wide_issue<1>(a, st[1], b, wave, lane, o, act_base);
        wide_stage<0>(st[0], R, wave, kq, rl);
        wait_vm_n<0>();
        __syncthreads();
        wide_issue<2>(a, st[0], b, wave, lane, o, act_base);
        wide_stage<1>(st[1], R, wave, kq, rl);
        wait_vm_n<0>();
        __syncthreads();
        wide_issue<3>(a, st[1], b, wave, lane, o, act_base);
        wide_stage<2>(st[0], R, wave, kq, rl);
        wait_vm_n<0>();
        __syncthreads();
        if (bi + 1 < nblk) wide_issue<0>(a, st[0], b + 1, wave, lane, o, act_base);
        wide_stage<3>(st[1], R, wave, kq, rl);
    }

    // Rows rw + 16 rt + 4 kq + i (pair p = rt, or p = matrix with GLU),
    // tokens t0 + 16 g + rl.
#pragma unroll
    for (int g = 0; g < 8; g++) {
        const int tok = t0 + 16 * g + rl;
        if (tok >= a.M) continue;
        const float us = *(const float *)(a.act + (int64_t)tok * a.act_stride + hact_unscale(a.n_in));
#pragma unroll
        for (int rt = 0; rt < RT; rt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = rw + 16 * rt + 4 * kq + i;
                if (r >= a.nrows) continue;
                const float v = R.acc[rt][g][i] * us;
                if (a.ks > 1) {
                    float *p = a.out + (((int64_t)blockIdx.z * 2) * a.M + tok) * a.nrows + r;
                    p[0] = v;
                    if (MODE == W_GLU) p[(int64_t)a.M * a.nrows] = R.acc[1][g][i] * us;
                } else {
                    const int64_t o2 = (int64_t)tok * a.ldy + r;
                    if (MODE == W_ADD) a.out[o2] = a.y_in[o2] + v;
                    else if (MODE == W_GLU) a.out[o2] = glu_act(v, R.acc[1][g][i] * us, a.gelu);
                    else a.out[o2] = v;
                }
            }
    }
}

// Splits of K (whole blocks) that give about two workgroups per CU.
int wide_splits(int64_t rows, int M, int nb, int cus, int mode) {
    const int64_t wgs = ((rows + wide_rows(mode) - 1) / wide_rows(mode)) * ((M + WG_TOK - 1) / WG_TOK);
    const int64_t want = (2 * (int64_t)cus + wgs / 2) / wgs;
    return (int)std::max<int64_t>(1, std::min<int64_t>({16, want, (int64_t)nb / 2}));
}

hipError_t launch_gemm_wide(const void *w, const void *w2, int64_t ne0, int64_t ne1, const void *act, int M, int mode,
                            float *y, const float *y_in, int64_t ldy, void *scratch, int ks, hipStream_t s) {
    WideArgs a{};
    a.gelu = (mode & GLU_GELU) ? 1 : 0;
    mode &= ~GLU_GELU;
    a.w = (const uint8_t *)w, a.w2 = (const uint8_t *)w2, a.act = (const uint8_t *)act;
    a.act_stride = (int64_t)hact_bytes(ne0), a.y_in = y_in, a.ldy = ldy;
    a.nrows = (int)ne1, a.nb = (int)(ne0 / 256), a.n_in = (int)ne0, a.M = M, a.ks = ks;
    a.out = ks > 1 ? (float *)scratch : y;
    const int rows = wide_rows(mode);
    const dim3 grid((unsigned)((M + WG_TOK - 1) / WG_TOK), (unsigned)((ne1 + rows - 1) / rows), (unsigned)ks);
    if (mode == W_GLU) hipLaunchKernelGGL(k_gemm_wide<W_GLU>, grid, dim3(256), 0, s, a);
    else if (mode == W_ADD) hipLaunchKernelGGL(k_gemm_wide<W_ADD>, grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(k_gemm_wide<W_STORE>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace ts5hip
