// The prompt matmul for Q4_K rows: Y[t] = W x_t for batches past 16 tokens
// (the reference's matmul_big path for prompts, engine/src/vk_backend.cpp:
// 866-918; its CPU restatement engine/src/cpu_backend.cpp:18-41).
//
// fp16 matrix cores with exact quants. A Q4_K weight is d*sc*q - dmin*m with
// q in 0..15, so per 32-value sub-block
//   y += d*sc * sum(q x) - dmin*m * sum(x)         (engine/src/quants.cpp:133-160)
// The quants are exact fp16 integers. The activations arrive as two fp16
// planes of x 2^-e (hi + lo, about 22 bits; the power of two keeps the
// residual stream's 1e11-sized values in range) with their 32-value sums X:
// one v_mfma_f32_16x16x32_f16 multiplies 16 rows x 32 quants by the hi plane
// of 16 tokens, a second adds the lo plane into the same fp32 accumulator,
// and the sub-block's scale and min are applied in fp32:
//   acc += d*sc * P - dmin*m * X;   y = acc * 2^e at the end.
//
// Workgroup: 4 waves, 128 rows x 64 tokens; wave w owns rows 32w..32w+31
// (2 row tiles) for all 4 token tiles. The K loop runs in stages of a quarter
// block (64 values, two sub-blocks). Every operand of a stage (the 64 tokens'
// hi/lo pieces and sums, the wave's quants and block headers) comes into LDS
// by DMA (global_load_lds_dwordx4), NS stages in flight: the loop itself
// issues no register loads, so the only waits are the explicit vmcnt ones.
// A token's 16 pieces of 16 bytes per stage sit at piece ^ (token & 15), so
// the 16 lanes that read one piece of 16 tokens hit 16 different bank groups.
// Split-K (grid z) when rows x tokens alone give too few workgroups; a second
// kernel adds the partial sums in a fixed order.
//
// Lane layout of the 16x16x32 MFMA: A lane l = row l%16, k-group l/16 (8
// values); B lane l = token l%16, the same k-group; D lane l = rows
// 4*(l/16)+i of token l%16. The k order inside the 32 only has to agree
// between A and B.
#include <algorithm>

#include "common.h"
#include "kernels.h"

namespace ts5hip {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

struct WideArgs {
    const uint8_t *w, *w2;  // Q4_K rows (w2: GLU's up projection)
    const uint8_t *act;     // M records of hact_bytes(n_in)
    int64_t act_stride;
    float *out;             // ks == 1: y [M][ldy]; ks > 1: partials [ks][2][M][nrows]
    const float *y_in;      // G_ADD: residual [M][ldy] (may be out)
    int64_t ldy;
    int nrows, nb, n_in, M, ks;
};

enum { W_STORE = 0, W_ADD = 1, W_GLU = 2 };
constexpr int WG_ROWS = 128, WG_TOK = 64;

template <int NW>
struct WideLds {
    static constexpr int NS = NW == 2 ? 2 : 3;  // stages in flight (GLU's are larger)
    static constexpr int PER = 6 + NW;          // DMA instructions per wave per stage
    struct Stage {
        uint4 b[WG_TOK * 16];    // [token][piece ^ (token & 15)]: hi pieces 0..7, lo 8..15
        float x[WG_TOK][2];      // the stage's two chunk sums per token
        uint4 wq[4][NW][32][2];  // [wave][matrix][row]: the 32 quant bytes of sub-blocks 2 q4, 2 q4 + 1
        uint4 wh[4][NW * 32];    // [wave][matrix * 32 + row]: block header (d, dmin, scales)
    } st[NS];
    float2 scl[4][NW][2][32];    // [wave][matrix][chunk][row]: (d sc, dmin m)
};

template <int NW>
__device__ inline void wide_issue(const WideArgs &a, typename WideLds<NW>::Stage &S, int sg, int wave, int lane,
                                  int r0, int t0) {
    const int b = sg >> 2, q4 = sg & 3;
#pragma unroll
    for (int i = 0; i < 4; i++) {  // activation pieces 64 j .. 64 j + 63
        const int j = 4 * wave + i, u = 64 * j + lane, tok = u >> 4, p = (u & 15) ^ (tok & 15);
        const uint8_t *src = a.act + (int64_t)min(t0 + tok, a.M - 1) * a.act_stride + (int64_t)b * 1024 +
                             (p >> 3) * 512 + q4 * 128 + (p & 7) * 16;
        dma16(src, lds_addr(S.b) + 1024 * j);
    }
    if (lane < 32) {  // chunk sums of tokens 16 wave .. +15
        const int tok = 16 * wave + (lane >> 1);
        const float *src = (const float *)(a.act + (int64_t)min(t0 + tok, a.M - 1) * a.act_stride + hact_x(a.n_in)) +
                           8 * b + 2 * q4 + (lane & 1);
        dma4(src, lds_addr(&S.x[16 * wave][0]));
    }
    const int rw = r0 + 32 * wave;
#pragma unroll
    for (int m = 0; m < NW; m++) {  // quants: lane = (row, 16-byte half)
        const int64_t row = min(rw + (lane >> 1), a.nrows - 1);
        const uint8_t *blk = (m ? a.w2 : a.w) + (row * a.nb + b) * Q4K_BYTES;
        dma16(blk + 16 + 32 * q4 + 16 * (lane & 1), lds_addr(&S.wq[wave][m][0][0]));
    }
    if (NW == 2 || lane < 32) {  // headers: lane = matrix * 32 + row
        const int64_t row = min(rw + (lane & 31), a.nrows - 1);
        const uint8_t *blk = ((lane >> 5) ? a.w2 : a.w) + (row * a.nb + b) * Q4K_BYTES;
        dma16(blk, lds_addr(&S.wh[wave][0]));
    }
}

// 8 quants (one nibble of each of 8 bytes) as exact fp16: byte -> 0x64bb is
// 1024 + q, less 1024.
__device__ inline v8h nib_f16(uint2 q, int hi) {
    const uint32_t v0 = (hi ? q.x >> 4 : q.x) & 0x0F0F0F0Fu, v1 = (hi ? q.y >> 4 : q.y) & 0x0F0F0F0Fu;
    const v2h k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    const v2h p0 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, v0, 0x04010400u)) - k1024;
    const v2h p1 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, v0, 0x04030402u)) - k1024;
    const v2h p2 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, v1, 0x04010400u)) - k1024;
    const v2h p3 = __builtin_bit_cast(v2h, __builtin_amdgcn_perm(0x64646464u, v1, 0x04030402u)) - k1024;
    return v8h{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void k_gemm_wide(WideArgs a) {
    constexpr int NW = MODE == W_GLU ? 2 : 1;
    using L = WideLds<NW>;
    constexpr int NS = L::NS, PER = L::PER;
    __shared__ L lds;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, kq = lane >> 4, rl = lane & 15;
    const int t0 = blockIdx.x * WG_TOK, r0 = blockIdx.y * WG_ROWS;
    const int total = a.nb * 4, sps = (total + a.ks - 1) / a.ks;
    const int s0 = blockIdx.z * sps, ns = max(0, min(total, s0 + sps) - s0);

    float acc[NW][2][4][4];
#pragma unroll
    for (int m = 0; m < NW; m++)
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
#pragma unroll
            for (int g = 0; g < 4; g++)
#pragma unroll
                for (int i = 0; i < 4; i++) acc[m][rt][g][i] = 0.f;

#pragma unroll
    for (int s = 0; s < NS - 1; s++)
        if (s < ns) wide_issue<NW>(a, lds.st[s], s0 + s, wave, lane, r0, t0);

    for (int s = 0; s < ns; s++) {
        // This wave's DMAs of stage s are done when at most the later stages' remain.
        if (NS == 3 && s + 1 < ns) wait_vm_n<PER>();
        else wait_vm_n<0>();
        __syncthreads();  // every wave's stage s is in; every wave is done with stage s - 1
        if (s + NS - 1 < ns) wide_issue<NW>(a, lds.st[(s + NS - 1) % NS], s0 + s + NS - 1, wave, lane, r0, t0);
        const typename L::Stage &S = lds.st[s % NS];
        const int q4 = (s0 + s) & 3;
        if (NW == 2 || lane < 32) {
            const uint4 h = S.wh[wave][lane];
            int sc0, m0, sc1, m1;
            kq_scale_min_pair(q4, h.y, h.z, h.w, sc0, m0, sc1, m1);
            const float d = h2f(h.x & 0xffff), dmin = h2f(h.x >> 16);
            lds.scl[wave][lane >> 5][0][lane & 31] = make_float2(d * (float)sc0, dmin * (float)m0);
            lds.scl[wave][lane >> 5][1][lane & 31] = make_float2(d * (float)sc1, dmin * (float)m1);
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int c = 0; c < 2; c++) {
            v8h A[NW][2];
            float ds[NW][2][4], dm[NW][2][4];
#pragma unroll
            for (int m = 0; m < NW; m++)
#pragma unroll
                for (int rt = 0; rt < 2; rt++) {
                    const uint2 q = *(const uint2 *)((const uint8_t *)&S.wq[wave][m][16 * rt + rl][0] + 8 * kq);
                    A[m][rt] = nib_f16(q, c);
                    const float4 sa = *(const float4 *)&lds.scl[wave][m][c][16 * rt + 4 * kq];
                    const float4 sb = *(const float4 *)&lds.scl[wave][m][c][16 * rt + 4 * kq + 2];
                    ds[m][rt][0] = sa.x, dm[m][rt][0] = sa.y, ds[m][rt][1] = sa.z, dm[m][rt][1] = sa.w;
                    ds[m][rt][2] = sb.x, dm[m][rt][2] = sb.y, ds[m][rt][3] = sb.z, dm[m][rt][3] = sb.w;
                }
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int tok = 16 * g + rl;
                const v8h bh = __builtin_bit_cast(v8h, S.b[16 * tok + ((4 * c + kq) ^ rl)]);
                const v8h bl = __builtin_bit_cast(v8h, S.b[16 * tok + ((8 + 4 * c + kq) ^ rl)]);
                const float X = S.x[tok][c];
#pragma unroll
                for (int m = 0; m < NW; m++)
#pragma unroll
                    for (int rt = 0; rt < 2; rt++) {
                        v4f P = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[m][rt], bh, v4f{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        P = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[m][rt], bl, P, 0, 0, 0);
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            acc[m][rt][g][i] = fmaf(ds[m][rt][i], P[i], fmaf(-dm[m][rt][i], X, acc[m][rt][g][i]));
                    }
            }
        }
    }

    // Rows r0 + 32 wave + 16 rt + 4 kq + i, tokens t0 + 16 g + rl.
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const int tok = t0 + 16 * g + rl;
        if (tok >= a.M) continue;
        const float us = *(const float *)(a.act + (int64_t)tok * a.act_stride + hact_unscale(a.n_in));
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = r0 + 32 * wave + 16 * rt + 4 * kq + i;
                if (r >= a.nrows) continue;
                const float v = acc[0][rt][g][i] * us;
                if (a.ks > 1) {
                    float *p = a.out + (((int64_t)blockIdx.z * 2) * a.M + tok) * a.nrows + r;
                    p[0] = v;
                    if (MODE == W_GLU) p[(int64_t)a.M * a.nrows] = acc[NW - 1][rt][g][i] * us;
                } else {
                    const int64_t o = (int64_t)tok * a.ldy + r;
                    if (MODE == W_ADD) a.out[o] = a.y_in[o] + v;
                    else if (MODE == W_GLU) a.out[o] = v / (1.0f + expf(-v)) * (acc[NW - 1][rt][g][i] * us);  // cpu_backend.cpp:260-261
                    else a.out[o] = v;
                }
            }
    }
}

int wide_splits(int64_t rows, int M, int nb, int cus) {
    const int64_t wgs = ((rows + WG_ROWS - 1) / WG_ROWS) * ((M + WG_TOK - 1) / WG_TOK);
    const int64_t want = (2 * (int64_t)cus + wgs / 2) / wgs;  // about two workgroups per CU
    return (int)std::max<int64_t>(1, std::min<int64_t>({16, want, (int64_t)nb / 2}));
}

hipError_t launch_gemm_wide(const void *w, const void *w2, int64_t ne0, int64_t ne1, const void *act, int M, int mode,
                            float *y, const float *y_in, int64_t ldy, void *scratch, int ks, hipStream_t s) {
    WideArgs a{};
    a.w = (const uint8_t *)w, a.w2 = (const uint8_t *)w2, a.act = (const uint8_t *)act;
    a.act_stride = (int64_t)hact_bytes(ne0), a.y_in = y_in, a.ldy = ldy;
    a.nrows = (int)ne1, a.nb = (int)(ne0 / 256), a.n_in = (int)ne0, a.M = M, a.ks = ks;
    a.out = ks > 1 ? (float *)scratch : y;
    const dim3 grid((unsigned)((M + WG_TOK - 1) / WG_TOK), (unsigned)((ne1 + WG_ROWS - 1) / WG_ROWS), (unsigned)ks);
    if (mode == W_GLU) hipLaunchKernelGGL(k_gemm_wide<W_GLU>, grid, dim3(256), 0, s, a);
    else if (mode == W_ADD) hipLaunchKernelGGL(k_gemm_wide<W_ADD>, grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL(k_gemm_wide<W_STORE>, grid, dim3(256), 0, s, a);
    return hipGetLastError();
}

}  // namespace ts5hip
