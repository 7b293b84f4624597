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

size_t gemm_act_bytes(uint32_t t, int64_t n) {
    return (t == T_Q8_0 || n % 256) ? act_bytes(n) : mact_bytes(n);
}

hipError_t launch_gemm_act(uint32_t t, const float *x, int64_t xstride, const float *w, float eps, int n, int ntok,
                           void *act, hipStream_t s) {
    if (t == T_Q8_0 || n % 256) return launch_act_quant(x, xstride, w, eps, n, ntok, act, s);
    hipLaunchKernelGGL(k_act_quant_m, dim3(ntok, (n / 16 + 255) / 256), dim3(256), 0, s, x, xstride, w, eps, n,
                       (uint8_t *)act, (int64_t)mact_bytes(n));
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float *x, const float *w, float eps, int n, int ntok, float *y, hipStream_t s) {
    if (n <= 256 * 16) hipLaunchKernelGGL(k_rmsnorm_reg<16>, dim3(ntok), dim3(256), 0, s, x, w, eps, n, y);
    else hipLaunchKernelGGL(k_rmsnorm, dim3(ntok), dim3(256), 0, s, x, w, eps, n, y);
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
