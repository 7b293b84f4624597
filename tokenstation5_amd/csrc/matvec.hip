// One-token k-quant matvecs y = W x for Q4_K, Q6_K and Q8_0 weights, and the
// fused gate/up + SiLU variant, against a quantized activation (Act).
//
// The reference computes y[r] = sum_i deq(W[r,i]) * x[i] with fp64
// accumulation (engine/src/cpu_backend.cpp:18-37); its GPU path reads 8
// lanes per Q4_K super-block with 16-byte loads (mv16_q4_k.glsl:64-113).
// Here the weights stay packed in registers: each lane takes whole 32-value
// sub-blocks, multiplies the raw quants with the activation's two int8 planes
// on v_dot4_i32_i8 (exact int32), and applies the block scales once per
// sub-block in fp32:
//   Q4_K: y += d*sc*(xs*sum q*x16) - dmin*m*(sum x)      (quants.cpp:140-157)
//   Q6_K: y += d*sc*xs*(sum q*x16 - 32*sum x16)          (quants.cpp:179-202)
//   Q8_0: y += d*xs*(sum q*x16)                          (quants.cpp:133-139)
// Bandwidth-bound: every weight byte is read once with dwordx4 loads; the
// activation (<= 36 KB) is re-read from L2 by every wave and reused across
// the R rows a wave owns. No MFMA.
#include "common.h"
#include "kernels.h"

namespace ts5hip {

// ---------------------------------------------------------------------------
// Formats. Each lane owns `sub` (0..LPB-1) of every block it visits; a wave
// covers BPI = 64 / LPB consecutive blocks of a row per iteration.
// ---------------------------------------------------------------------------
struct WPtr {
    const uint8_t *body;     // blocks (Q4_K: whole blocks; Q6_K/Q8_0: bodies)
    const uint16_t *dscale;  // f16 block scales of split layouts
};

__device__ inline WPtr wptr(uint32_t t, const void *w, int64_t nblocks) {
    WPtr p;
    p.body = (const uint8_t *)w;
    p.dscale = (t == T_Q6_K || t == T_Q8_0) ? (const uint16_t *)(p.body + split_scale_offset(t, nblocks)) : nullptr;
    return p;
}

__device__ inline uint4 ld16(const void *p) { return *(const uint4 *)p; }

// Q4_K: 4 lanes per block, lane `sub` = nibble group g: sub-blocks 2g (low
// nibbles) and 2g+1 (high nibbles), 64 values.
struct Q4K {
    static constexpr int LPB = 4;
    struct X {
        uint4 h[4], l[4];
        float s0, s1, m0, m1;
    };
    struct W {
        uint4 hdr, qa, qb;
    };
    __device__ static X load_x(const CAct &x, int b, int sub) {
        X r;
        const int base = b * 256 + 64 * sub;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            r.h[k] = ld16(x.hi + base + 16 * k);
            r.l[k] = ld16(x.lo + base + 16 * k);
        }
        const int s = b * 8 + 2 * sub;
        r.s0 = x.scale[s];
        r.s1 = x.scale[s + 1];
        r.m0 = x.sum[s];
        r.m1 = x.sum[s + 1];
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
        const uint32_t xh0[8] = {x.h[0].x, x.h[0].y, x.h[0].z, x.h[0].w, x.h[1].x, x.h[1].y, x.h[1].z, x.h[1].w};
        const uint32_t xh1[8] = {x.h[2].x, x.h[2].y, x.h[2].z, x.h[2].w, x.h[3].x, x.h[3].y, x.h[3].z, x.h[3].w};
        const uint32_t xl0[8] = {x.l[0].x, x.l[0].y, x.l[0].z, x.l[0].w, x.l[1].x, x.l[1].y, x.l[1].z, x.l[1].w};
        const uint32_t xl1[8] = {x.l[2].x, x.l[2].y, x.l[2].z, x.l[2].w, x.l[3].x, x.l[3].y, x.l[3].z, x.l[3].w};
        int ah0 = 0, al0 = 0, ah1 = 0, al1 = 0;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int lo = (int)(q[k] & 0x0F0F0F0Fu), hi = (int)((q[k] >> 4) & 0x0F0F0F0Fu);
            ah0 = dot4(lo, (int)xh0[k], ah0);
            al0 = dot4(lo, (int)xl0[k], al0);
            ah1 = dot4(hi, (int)xh1[k], ah1);
            al1 = dot4(hi, (int)xl1[k], al1);
        }
        int sc0, m0, sc1, m1;
        kq_scale_min(2 * sub, w.hdr.y, w.hdr.z, w.hdr.w, sc0, m0);
        kq_scale_min(2 * sub + 1, w.hdr.y, w.hdr.z, w.hdr.w, sc1, m1);
        const float d = h2f(w.hdr.x & 0xffff), dmin = h2f(w.hdr.x >> 16);
        const float p = (float)sc0 * x.s0 * (float)(ah0 * 256 + al0) + (float)sc1 * x.s1 * (float)(ah1 * 256 + al1);
        return d * p - dmin * ((float)m0 * x.m0 + (float)m1 * x.m1);
    }
};

// Q6_K: 4 lanes per block, lane `sub` = (half h = sub/2, i0 = 16*(sub%2)):
// the four 16-value runs at 128h + 32c + i0 (c = 0..3), 64 values.
struct Q6K {
    static constexpr int LPB = 4;
    struct X {
        uint32_t h[4][4], l[4][4];  // [run c][dword]
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
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int base = b * 256 + 128 * h + 32 * c + i0;
            const uint4 vh = ld16(x.hi + base), vl = ld16(x.lo + base);
            r.h[c][0] = vh.x, r.h[c][1] = vh.y, r.h[c][2] = vh.z, r.h[c][3] = vh.w;
            r.l[c][0] = vl.x, r.l[c][1] = vl.y, r.l[c][2] = vl.z, r.l[c][3] = vl.w;
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
        int ah[4] = {0, 0, 0, 0}, al[4] = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t q0 = (qa[k] & 0x0F0F0F0Fu) | ((qh[k] << 4) & 0x30303030u);
            const uint32_t q1 = (qb[k] & 0x0F0F0F0Fu) | ((qh[k] << 2) & 0x30303030u);
            const uint32_t q2 = ((qa[k] >> 4) & 0x0F0F0F0Fu) | (qh[k] & 0x30303030u);
            const uint32_t q3 = ((qb[k] >> 4) & 0x0F0F0F0Fu) | ((qh[k] >> 2) & 0x30303030u);
            ah[0] = dot4((int)q0, (int)x.h[0][k], ah[0]);
            al[0] = dot4((int)q0, (int)x.l[0][k], al[0]);
            ah[1] = dot4((int)q1, (int)x.h[1][k], ah[1]);
            al[1] = dot4((int)q1, (int)x.l[1][k], al[1]);
            ah[2] = dot4((int)q2, (int)x.h[2][k], ah[2]);
            al[2] = dot4((int)q2, (int)x.l[2][k], al[2]);
            ah[3] = dot4((int)q3, (int)x.h[3][k], ah[3]);
            al[3] = dot4((int)q3, (int)x.l[3][k], al[3]);
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
            const int v = ah[c] * 256 + al[c] - 32 * x.is[c];
            p += (float)sc * x.s[c] * (float)v;
        }
        return w.d * p;
    }
};

// Q8_0: 2 lanes per 32-value block, 16 values each.
struct Q80 {
    static constexpr int LPB = 2;
    struct X {
        uint4 h, l;
        float s;
    };
    struct W {
        uint4 q;
        float d;
    };
    __device__ static X load_x(const CAct &x, int b, int sub) {
        X r;
        r.h = ld16(x.hi + b * 32 + 16 * sub);
        r.l = ld16(x.lo + b * 32 + 16 * sub);
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
        int ah = 0, al = 0;
        ah = dot4((int)w.q.x, (int)x.h.x, ah);
        ah = dot4((int)w.q.y, (int)x.h.y, ah);
        ah = dot4((int)w.q.z, (int)x.h.z, ah);
        ah = dot4((int)w.q.w, (int)x.h.w, ah);
        al = dot4((int)w.q.x, (int)x.l.x, al);
        al = dot4((int)w.q.y, (int)x.l.y, al);
        al = dot4((int)w.q.z, (int)x.l.z, al);
        al = dot4((int)w.q.w, (int)x.l.w, al);
        return w.d * x.s * (float)(ah * 256 + al);
    }
};

// ---------------------------------------------------------------------------
// y[r] (=|+=) W[r] . x for the R rows of each wave. The last wave's surplus
// rows re-read the final row (in bounds) and are not written.
// ---------------------------------------------------------------------------
enum { EPI_STORE = 0, EPI_ADD = 1 };

template <class F, int R>
__device__ inline void mv_rows(const WPtr &w, int64_t row0, int64_t nrows, int nb, const CAct &x, float (&acc)[R]) {
    constexpr int BPI = WAVE / F::LPB;
    const int lane = threadIdx.x & 63, bsub = lane / F::LPB, sub = lane % F::LPB;
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = 0.f;
    for (int b = bsub; b < nb; b += BPI) {
        const typename F::X xf = F::load_x(x, b, sub);
        typename F::W wf[R];
#pragma unroll
        for (int r = 0; r < R; r++) wf[r] = F::load_w(w, min(row0 + r, nrows - 1), nb, b, sub);
#pragma unroll
        for (int r = 0; r < R; r++) acc[r] += F::dot(wf[r], xf, sub);
    }
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = wave_sum(acc[r]);
}

template <class F, int R, int WAVES, int EPI>
__global__ __launch_bounds__(WAVES *WAVE) void k_mv(uint32_t t, const void *__restrict__ W, int64_t nrows, int nb,
                                                    const uint8_t *__restrict__ actp, int n_in, float *__restrict__ y) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row0 = ((int64_t)blockIdx.x * WAVES + wave) * R;
    if (row0 >= nrows) return;
    const WPtr w = wptr(t, W, (int64_t)nb * nrows);
    const CAct x = cact_view(actp, n_in);
    float acc[R];
    mv_rows<F, R>(w, row0, nrows, nb, x, acc);
    if (lane < R && row0 + lane < nrows) {
        float v = acc[0];
#pragma unroll
        for (int r = 1; r < R; r++)
            if (lane == r) v = acc[r];
        if (EPI == EPI_ADD)
            y[row0 + lane] += v;
        else
            y[row0 + lane] = v;
    }
}

// Fused gate/up: out[r] = silu(gate[r] . x) * (up[r] . x) (the reference's
// float expression g / (1 + exp(-g)) * u, engine/src/cpu_backend.cpp:260-261),
// written as fp32 (optional) and as the Act of the next matvec (one 32-row
// sub-block per workgroup, so R * WAVES == 32).
template <class F, int R, int WAVES>
__global__ __launch_bounds__(WAVES *WAVE) void k_mv_glu(uint32_t t, const void *__restrict__ Wg,
                                                        const void *__restrict__ Wu, int64_t nrows, int nb,
                                                        const uint8_t *__restrict__ actp, int n_in,
                                                        float *__restrict__ y, uint8_t *__restrict__ act_out) {
    static_assert(R * WAVES == 32, "one 32-row sub-block per workgroup");
    __shared__ float outv[32];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t row0 = ((int64_t)blockIdx.x * WAVES + wave) * R;
    const WPtr wg = wptr(t, Wg, (int64_t)nb * nrows), wu = wptr(t, Wu, (int64_t)nb * nrows);
    const CAct x = cact_view(actp, n_in);
    float g[R], u[R];
    mv_rows<F, R>(wg, row0, nrows, nb, x, g);
    mv_rows<F, R>(wu, row0, nrows, nb, x, u);
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; r++) outv[wave * R + r] = g[r] / (1.0f + expf(-g[r])) * u[r];
    }
    __syncthreads();
    if (threadIdx.x < 32) {
        const float v = outv[threadIdx.x];
        const int64_t row = (int64_t)blockIdx.x * 32 + threadIdx.x;
        if (y) y[row] = v;
        quant32(v, threadIdx.x, act_view(act_out, nrows), blockIdx.x);
    }
}

// ---------------------------------------------------------------------------
// Launchers. Shapes are checked by the caller (capi.cpp).
// ---------------------------------------------------------------------------
template <class F, int R, int WAVES>
static hipError_t mv_launch(uint32_t t, const void *w, int64_t ne0, int64_t ne1, const void *act, float *y, int add,
                            hipStream_t s) {
    const int nb = (int)(ne0 / block_values(t));
    const int64_t rows_per_wg = (int64_t)R * WAVES;
    const dim3 grid((unsigned)((ne1 + rows_per_wg - 1) / rows_per_wg));
    if (add)
        hipLaunchKernelGGL((k_mv<F, R, WAVES, EPI_ADD>), grid, dim3(WAVES * WAVE), 0, s, t, w, ne1, nb,
                           (const uint8_t *)act, (int)ne0, y);
    else
        hipLaunchKernelGGL((k_mv<F, R, WAVES, EPI_STORE>), grid, dim3(WAVES * WAVE), 0, s, t, w, ne1, nb,
                           (const uint8_t *)act, (int)ne0, y);
    return hipGetLastError();
}

hipError_t launch_matvec(uint32_t t, const void *w, int64_t ne0, int64_t ne1, const void *act, float *y, int add,
                         hipStream_t s) {
    switch (t) {
    case T_Q4_K: return mv_launch<Q4K, 4, 4>(t, w, ne0, ne1, act, y, add, s);
    case T_Q6_K: return mv_launch<Q6K, 4, 4>(t, w, ne0, ne1, act, y, add, s);
    case T_Q8_0: return mv_launch<Q80, 4, 4>(t, w, ne0, ne1, act, y, add, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_matvec_glu(uint32_t t, const void *wg, const void *wu, int64_t ne0, int64_t ne1, const void *act,
                             float *y, void *act_out, hipStream_t s) {
    const int nb = (int)(ne0 / block_values(t));
    const dim3 grid((unsigned)(ne1 / 32));
    switch (t) {
    case T_Q4_K:
        hipLaunchKernelGGL((k_mv_glu<Q4K, 4, 8>), grid, dim3(8 * WAVE), 0, s, t, wg, wu, ne1, nb, (const uint8_t *)act,
                           (int)ne0, y, (uint8_t *)act_out);
        return hipGetLastError();
    case T_Q6_K:
        hipLaunchKernelGGL((k_mv_glu<Q6K, 4, 8>), grid, dim3(8 * WAVE), 0, s, t, wg, wu, ne1, nb, (const uint8_t *)act,
                           (int)ne0, y, (uint8_t *)act_out);
        return hipGetLastError();
    case T_Q8_0:
        hipLaunchKernelGGL((k_mv_glu<Q80, 4, 8>), grid, dim3(8 * WAVE), 0, s, t, wg, wu, ne1, nb, (const uint8_t *)act,
                           (int)ne0, y, (uint8_t *)act_out);
        return hipGetLastError();
    }
    return hipErrorInvalidValue;
}

}  // namespace ts5hip
