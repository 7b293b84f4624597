// RMSNorm (engine/src/cpu_backend.cpp:48-53) and the quantized-activation
// form every matvec reads (see Act in common.h).
#include "common.h"
#include "kernels.h"
#include "mv_core.h"

namespace ts5hip {

// Block-wide sum over a 256-thread block (4 waves).
__device__ inline float block_sum256(float v, float *red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) red[w] = v;
    __syncthreads();
    v = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    return v;
}

// 1 / sqrt(mean(x^2) + eps) of one token's n values (the reference keeps
// the sum in double; fp32 over <= 16384 values is within 1e-6 relative).
__device__ inline float rms_scale(const float *x, int n, float eps, float *red) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
    ss = block_sum256(ss, red);
    return 1.0f / sqrtf(ss / (float)n + eps);
}

// y = x * s * w per token (blockIdx.x); 256 threads.
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, float eps,
                                                 int n, float *__restrict__ y) {
    __shared__ float red[4];
    const float *xt = x + (int64_t)blockIdx.x * n;
    float *yt = y + (int64_t)blockIdx.x * n;
    const float s = rms_scale(xt, n, eps, red);
    for (int i = threadIdx.x; i < n; i += blockDim.x) yt[i] = xt[i] * s * w[i];
}

// Gemma 3's norm after attention / the FFN, then the residual add
// (engine/src/cpu_backend.cpp:250-252, :263-265): x_t += rmsnorm(o_t) * w for
// token blockIdx.x; rows of at most 256 * PER values held in registers.
template <int PER>
__global__ __launch_bounds__(256) void k_norm_add(const float *__restrict__ o, int64_t ostride,
                                                  const float *__restrict__ w, float eps, int n, float *x,
                                                  int64_t xstride) {
    __shared__ float red[4];
    const float *ot = o + (int64_t)blockIdx.x * ostride;
    float *xt = x + (int64_t)blockIdx.x * xstride;
    float v[PER], ss = 0.f;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = threadIdx.x + 256 * k;
        v[k] = i < n ? ot[i] : 0.f;
        ss += v[k] * v[k];
    }
    const float sc = 1.0f / sqrtf(block_sum256(ss, red) / (float)n + eps);
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = threadIdx.x + 256 * k;
        if (i < n) xt[i] += v[k] * sc * w[i];
    }
}

// Act of x (optionally rms-normalised by w first): token blockIdx.x, 16-runs
// 256*blockIdx.y .. +255 (one per thread; the norm's sum over the whole row
// is taken by every slice).
__global__ __launch_bounds__(256) void k_act_quant(const float *__restrict__ x, int64_t xstride,
                                                   const float *__restrict__ w, float eps, int n,
                                                   uint8_t *__restrict__ act, int64_t act_stride) {
    __shared__ float red[4];
    const float *xt = x + (int64_t)blockIdx.x * xstride;
    const Act a = act_view(act + (int64_t)blockIdx.x * act_stride, n);
    const float s = act_rms<256>(xt, w, eps, n, red);
    const int r0 = 256 * blockIdx.y;
    act_runs<256>(xt, w, s, r0, min(n / 16, r0 + 256), a);
}

// The same in one pass over x for rows of at most 256 * PER values: thread t
// holds values t, t + 256, ... in registers between the norm's sum and the
// scaled write, so each row is read from memory once.
template <int PER>
__global__ __launch_bounds__(256) void k_rmsnorm_reg(const float *__restrict__ x, const float *__restrict__ w,
                                                     float eps, int n, float *__restrict__ y) {
    __shared__ float red[4];
    const float *xt = x + (int64_t)blockIdx.x * n;
    float *yt = y + (int64_t)blockIdx.x * n;
    float v[PER], ss = 0.f;
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = threadIdx.x + 256 * k;
        v[k] = i < n ? xt[i] : 0.f;
        ss += v[k] * v[k];
    }
    const float s = 1.0f / sqrtf(block_sum256(ss, red) / (float)n + eps);
#pragma unroll
    for (int k = 0; k < PER; k++) {
        const int i = threadIdx.x + 256 * k;
        if (i < n) yt[i] = v[k] * s * w[i];
    }
}

// The matmul layout (MAct) of x, optionally rms-normalised: token blockIdx.x,
// 16-runs 256*blockIdx.y .. +255 (one per thread).
__global__ __launch_bounds__(256) void k_act_quant_m(const float *__restrict__ x, int64_t xstride,
                                                     const float *__restrict__ w, float eps, int n,
                                                     uint8_t *__restrict__ act, int64_t act_stride) {
    __shared__ float red[4];
    const float *xt = x + (int64_t)blockIdx.x * xstride;
    uint8_t *m = act + (int64_t)blockIdx.x * act_stride;
    const float s = act_rms<256>(xt, w, eps, n, red);
    const int r = 256 * blockIdx.y + threadIdx.x;  // runs 2g, 2g+1 in adjacent lanes, both in or out
    if (r >= n / 16) return;
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const float4 f = *(const float4 *)(xt + 16 * r + 4 * k);
        v[4 * k] = f.x, v[4 * k + 1] = f.y, v[4 * k + 2] = f.z, v[4 * k + 3] = f.w;
    }
    if (w) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float4 g = *(const float4 *)(w + 16 * r + 4 * k);
            v[4 * k] = v[4 * k] * s * g.x;
            v[4 * k + 1] = v[4 * k + 1] * s * g.y;
            v[4 * k + 2] = v[4 * k + 2] * s * g.z;
            v[4 * k + 3] = v[4 * k + 3] * s * g.w;
        }
    }
    quant_run_m(v, r, m);
}

// The prompt matmuls' fp16 pair form (hact_*) of x, optionally
// rms-normalised: token blockIdx.x; the largest |value| sets the token's power
// of two, then each thread writes 32-value chunks (hi, lo and their sum).
__global__ __launch_bounds__(256) void k_act_half(const float *__restrict__ x, int64_t xstride,
                                                  const float *__restrict__ w, float eps, int n,
                                                  uint8_t *__restrict__ act, int64_t act_stride) {
    __shared__ float red[4], redm[4];
    const float *xt = x + (int64_t)blockIdx.x * xstride;
    uint8_t *o = act + (int64_t)blockIdx.x * act_stride;
    const float s = act_rms<256>(xt, w, eps, n, red);
    auto value4 = [&](int i) {
        float4 v = *(const float4 *)(xt + i);
        if (w) {
            const float4 g = *(const float4 *)(w + i);
            v.x = v.x * s * g.x, v.y = v.y * s * g.y, v.z = v.z * s * g.z, v.w = v.w * s * g.w;
        }
        return v;
    };
    float amax = 0.f;
    for (int i = 4 * threadIdx.x; i < n; i += 1024) {
        const float4 v = value4(i);
        amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) redm[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
    const int e = amax > 0.f ? max(ilogbf(amax) - 13, -100) : 0;  // amax 2^-e in [2^13, 2^14)
    const float scale = ldexpf(1.0f, -e);
    if (threadIdx.x == 0) *(float *)(o + hact_unscale(n)) = ldexpf(1.0f, e);
    for (int c = threadIdx.x; c < n / 32; c += 256) {
        uint32_t hw[16], lw[16];
        float sum = 0.f;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const float4 v = value4(32 * c + 4 * k);
            const float f[4] = {v.x * scale, v.y * scale, v.z * scale, v.w * scale};
#pragma unroll
            for (int j = 0; j < 4; j += 2) {
                const _Float16 h0 = (_Float16)f[j], h1 = (_Float16)f[j + 1];
                const _Float16 l0 = (_Float16)(f[j] - (float)h0), l1 = (_Float16)(f[j + 1] - (float)h1);
                hw[2 * k + j / 2] = __builtin_bit_cast(uint16_t, h0) | (uint32_t)__builtin_bit_cast(uint16_t, h1) << 16;
                lw[2 * k + j / 2] = __builtin_bit_cast(uint16_t, l0) | (uint32_t)__builtin_bit_cast(uint16_t, l1) << 16;
                sum += f[j] + f[j + 1];
            }
        }
        uint8_t *blk = o + (size_t)(c / 8) * 1024 + (c % 8) * 64;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            ((uint4 *)blk)[k] = make_uint4(hw[4 * k], hw[4 * k + 1], hw[4 * k + 2], hw[4 * k + 3]);
            ((uint4 *)(blk + 512))[k] = make_uint4(lw[4 * k], lw[4 * k + 1], lw[4 * k + 2], lw[4 * k + 3]);
        }
        const float xs = sum * (1.0f / 32);  // exact; keeps the sums in fp16 range
        const _Float16 xh = (_Float16)xs, xl = (_Float16)(xs - (float)xh);
        uint16_t *xq = (uint16_t *)(o + hact_x(n)) + 4 * (c / 2) + (c & 1);  // [quarter][hi pair, lo pair]
        xq[0] = __builtin_bit_cast(uint16_t, xh);
        xq[2] = __builtin_bit_cast(uint16_t, xl);
    }
}

// The same form from one read of x: thread t holds 16-value runs t, t + 256,
// ... (at most RUNS) in registers through the norm's sum, the maximum and the
// writes; the two runs of a 32-value chunk sit in adjacent lanes.
template <int RUNS>
__global__ __launch_bounds__(256) void k_act_half_reg(const float *__restrict__ x, int64_t xstride,
                                                      const float *__restrict__ w, float eps, int n,
                                                      uint8_t *__restrict__ act, int64_t act_stride) {
    __shared__ float red[4], redm[4];
    const float *xt = x + (int64_t)blockIdx.x * xstride;
    uint8_t *o = act + (int64_t)blockIdx.x * act_stride;
    const int tid = threadIdx.x, nr = n / 16;
    float v[RUNS][16];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < RUNS; k++) {
        const int r = tid + 256 * k;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float4 f = r < nr ? *(const float4 *)(xt + 16 * r + 4 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
            v[k][4 * j] = f.x, v[k][4 * j + 1] = f.y, v[k][4 * j + 2] = f.z, v[k][4 * j + 3] = f.w;
            ss += f.x * f.x + f.y * f.y + f.z * f.z + f.w * f.w;
        }
    }
    float s = 1.0f;
    if (w) {  // the same expression as act_rms
        ss = wave_sum(ss);
        if ((tid & 63) == 0) red[tid >> 6] = ss;
        __syncthreads();
        s = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)n + eps);
    }
    float amax = 0.f;
#pragma unroll
    for (int k = 0; k < RUNS; k++) {
        const int r = tid + 256 * k;
        if (w && r < nr) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 g = *(const float4 *)(w + 16 * r + 4 * j);
                v[k][4 * j] = v[k][4 * j] * s * g.x, v[k][4 * j + 1] = v[k][4 * j + 1] * s * g.y;
                v[k][4 * j + 2] = v[k][4 * j + 2] * s * g.z, v[k][4 * j + 3] = v[k][4 * j + 3] * s * g.w;
            }
        }
#pragma unroll
        for (int i = 0; i < 16; i++) amax = fmaxf(amax, fabsf(v[k][i]));
    }
    amax = wave_max(amax);
    if ((tid & 63) == 0) redm[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
    const int e = amax > 0.f ? max(ilogbf(amax) - 13, -100) : 0;  // amax 2^-e in [2^13, 2^14)
    const float scale = ldexpf(1.0f, -e);
    if (tid == 0) *(float *)(o + hact_unscale(n)) = ldexpf(1.0f, e);
#pragma unroll
    for (int k = 0; k < RUNS; k++) {
        const int r = tid + 256 * k;  // runs 2c, 2c + 1 in adjacent lanes, both in or both out
        uint32_t hw[8], lw[8];
        float sum = 0.f;
#pragma unroll
        for (int j = 0; j < 16; j += 2) {
            const float f0 = v[k][j] * scale, f1 = v[k][j + 1] * scale;
            const _Float16 h0 = (_Float16)f0, h1 = (_Float16)f1;
            const _Float16 l0 = (_Float16)(f0 - (float)h0), l1 = (_Float16)(f1 - (float)h1);
            hw[j / 2] = __builtin_bit_cast(uint16_t, h0) | (uint32_t)__builtin_bit_cast(uint16_t, h1) << 16;
            lw[j / 2] = __builtin_bit_cast(uint16_t, l0) | (uint32_t)__builtin_bit_cast(uint16_t, l1) << 16;
            sum += f0 + f1;
        }
        sum += __shfl_xor(sum, 1, WAVE);
        if (r >= nr) continue;
        const int c = r / 2;  // the 32-value chunk
        uint8_t *blk = o + (size_t)(c / 8) * 1024 + (c % 8) * 64 + (r & 1) * 32;
        ((uint4 *)blk)[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        ((uint4 *)blk)[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
        ((uint4 *)(blk + 512))[0] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        ((uint4 *)(blk + 512))[1] = make_uint4(lw[4], lw[5], lw[6], lw[7]);
        if ((r & 1) == 0) {
            const float xs = sum * (1.0f / 32);
            const _Float16 xh = (_Float16)xs, xl = (_Float16)(xs - (float)xh);
            uint16_t *xq = (uint16_t *)(o + hact_x(n)) + 4 * (c / 2) + (c & 1);
            xq[0] = __builtin_bit_cast(uint16_t, xh);
            xq[2] = __builtin_bit_cast(uint16_t, xl);
        }
    }
}

size_t gemm_act_bytes(uint32_t t, int64_t n, int ntok) {
    switch (gemm_act_form(t, n, ntok)) {
    case GA_HACT: return hact_bytes(n);
    case GA_MACT: return mact_bytes(n);
    default: return act_bytes(n);
    }
}

hipError_t launch_gemm_act(uint32_t t, const float *x, int64_t xstride, const float *w, float eps, int n, int ntok,
                           void *act, hipStream_t s) {
    const int form = gemm_act_form(t, n, ntok);
    if (form == GA_ACT) return launch_act_quant(x, xstride, w, eps, n, ntok, act, s);
    if (form == GA_HACT && n <= 256 * 16)
        hipLaunchKernelGGL(k_act_half_reg<1>, dim3(ntok), dim3(256), 0, s, x, xstride, w, eps, n, (uint8_t *)act,
                           (int64_t)hact_bytes(n));
    else if (form == GA_HACT && n <= 256 * 64)
        hipLaunchKernelGGL(k_act_half_reg<4>, dim3(ntok), dim3(256), 0, s, x, xstride, w, eps, n, (uint8_t *)act,
                           (int64_t)hact_bytes(n));
    else if (form == GA_HACT)
        hipLaunchKernelGGL(k_act_half, dim3(ntok), dim3(256), 0, s, x, xstride, w, eps, n, (uint8_t *)act,
                           (int64_t)hact_bytes(n));
    else
        hipLaunchKernelGGL(k_act_quant_m, dim3(ntok, (n / 16 + 255) / 256), dim3(256), 0, s, x, xstride, w, eps, n,
                           (uint8_t *)act, (int64_t)mact_bytes(n));
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, const float *w, float eps, int n, int ntok, float *y, hipStream_t s) {
    if (n <= 256 * 16) hipLaunchKernelGGL(k_rmsnorm_reg<16>, dim3(ntok), dim3(256), 0, s, x, w, eps, n, y);
    else hipLaunchKernelGGL(k_rmsnorm, dim3(ntok), dim3(256), 0, s, x, w, eps, n, y);
    return hipGetLastError();
}

hipError_t launch_norm_add(const float *o, int64_t ostride, const float *w, float eps, int n, int ntok, float *x,
                           int64_t xstride, hipStream_t s) {
    if (n <= 256 * 8) hipLaunchKernelGGL(k_norm_add<8>, dim3(ntok), dim3(256), 0, s, o, ostride, w, eps, n, x, xstride);
    else if (n <= 256 * 16) hipLaunchKernelGGL(k_norm_add<16>, dim3(ntok), dim3(256), 0, s, o, ostride, w, eps, n, x, xstride);
    else if (n <= 256 * 32) hipLaunchKernelGGL(k_norm_add<32>, dim3(ntok), dim3(256), 0, s, o, ostride, w, eps, n, x, xstride);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_act_quant(const float *x, int64_t xstride, const float *w, float eps, int n, int ntok, void *act,
                            hipStream_t s) {
    hipLaunchKernelGGL(k_act_quant, dim3(ntok, (n / 16 + 255) / 256), dim3(256), 0, s, x, xstride, w, eps, n,
                       (uint8_t *)act,
                       (int64_t)act_bytes(n));
    return hipGetLastError();
}

}  // namespace ts5hip
