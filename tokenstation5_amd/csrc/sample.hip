// Reductions over the logits for sampling (Engine::sample,
// engine/src/engine.cpp:16-46): greedy argmax with the first maximum winning
// (std::max_element), and the top k (k <= 64) sorted by descending logit,
// ties by ascending id, for the host's top-p / discrete_distribution draw.
#include <climits>

#include "common.h"
#include "kernels.h"

namespace ts5hip {

constexpr int ARGMAX_WG = 256;

// (v, i) ranks before (w, j): larger value, then smaller id.
__device__ inline bool before(float v, int i, float w, int j) { return v > w || (v == w && i < j); }

__device__ inline void wave_best(float &v, int &i) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float w = __shfl_xor(v, o, WAVE);
        const int j = __shfl_xor(i, o, WAVE);
        if (before(w, j, v, i)) v = w, i = j;
    }
}

__device__ inline void block_best(float &v, int &i, float *vs, int *is) {
    wave_best(v, i);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    if (lane == 0) vs[w] = v, is[w] = i;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < (int)(blockDim.x >> 6); k++)
            if (before(vs[k], is[k], v, i)) v = vs[k], i = is[k];
    }
}

// grid ARGMAX_WG x 256 threads over rows of n logits (blockIdx.y = row).
__global__ __launch_bounds__(256) void k_argmax_part(const float *__restrict__ x, int n, float *__restrict__ pv,
                                                     int *__restrict__ pi) {
    __shared__ float vs[4];
    __shared__ int is[4];
    const float *xr = x + (int64_t)blockIdx.y * n;
    float v = -INFINITY;
    int i = INT_MAX;
    for (int k = blockIdx.x * 256 + threadIdx.x; k < n; k += gridDim.x * 256) {
        const float w = xr[k];
        if (before(w, k, v, i)) v = w, i = k;
    }
    block_best(v, i, vs, is);
    if (threadIdx.x == 0) {
        pv[blockIdx.y * gridDim.x + blockIdx.x] = v;
        pi[blockIdx.y * gridDim.x + blockIdx.x] = i;
    }
}

// One block per row. Writes out[row]; when `seq` is given (the device-side
// greedy loop, one row) also stores the id as the next position's token,
// seq[*pos + 1], and advances *pos.
__global__ __launch_bounds__(256) void k_argmax_final(const float *__restrict__ pv, const int *__restrict__ pi, int np,
                                                      int32_t *__restrict__ out, int32_t *__restrict__ seq,
                                                      int32_t *__restrict__ pos) {
    __shared__ float vs[4];
    __shared__ int is[4];
    float v = -INFINITY;
    int i = INT_MAX;
    for (int k = threadIdx.x; k < np; k += 256) {
        const float w = pv[blockIdx.x * np + k];
        const int j = pi[blockIdx.x * np + k];
        if (before(w, j, v, i)) v = w, i = j;
    }
    block_best(v, i, vs, is);
    if (threadIdx.x == 0) {
        if (i == INT_MAX) i = 0;  // every logit NaN
        out[blockIdx.x] = i;
        if (seq) {
            const int p = *pos;
            seq[p + 1] = i;
            *pos = p + 1;
        }
    }
}

// ---------------------------------------------------------------------------
// Top-k: each of TOPK_WG workgroups sorts its slice (<= 2048 logits) in LDS
// with a bitonic network and keeps its best k; one workgroup then sorts the
// TOPK_WG * k candidates (<= 8192, 64 KB of LDS).
// ---------------------------------------------------------------------------
constexpr int TOPK_WG = 128, TOPK_SLICE = 2048, TOPK_MAX = 64;

template <int N>
__device__ inline void bitonic(float *v, int *ix) {
    for (int size = 2; size <= N; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int t = threadIdx.x; t < N / 2; t += blockDim.x) {
                const int lo = 2 * t - (t & (stride - 1)), hi = lo + stride;
                const bool desc = (lo & size) == 0;  // first half of each run sorts "best first"
                const bool swap = desc ? before(v[hi], ix[hi], v[lo], ix[lo]) : before(v[lo], ix[lo], v[hi], ix[hi]);
                if (swap) {
                    const float tv = v[lo];
                    v[lo] = v[hi];
                    v[hi] = tv;
                    const int ti = ix[lo];
                    ix[lo] = ix[hi];
                    ix[hi] = ti;
                }
            }
        }
    }
    __syncthreads();
}

// grid (TOPK_WG, rows): workgroup x of row y sorts its slice of that row.
__global__ __launch_bounds__(256) void k_topk_part(const float *__restrict__ x, int n, int k, float *__restrict__ cv,
                                                   int *__restrict__ ci) {
    __shared__ float v[TOPK_SLICE];
    __shared__ int ix[TOPK_SLICE];
    const float *xr = x + (int64_t)blockIdx.y * n;
    const int per = (n + gridDim.x - 1) / gridDim.x;
    const int lo = blockIdx.x * per;
    for (int t = threadIdx.x; t < TOPK_SLICE; t += 256) {
        const int g = lo + t;
        const bool ok = t < per && g < n;
        v[t] = ok ? xr[g] : -INFINITY;
        ix[t] = ok ? g : INT_MAX;
    }
    bitonic<TOPK_SLICE>(v, ix);
    const int64_t o = ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * k;
    for (int t = threadIdx.x; t < k; t += 256) {
        cv[o + t] = v[t];
        ci[o + t] = ix[t];
    }
}

// One workgroup per row: the row's TOPK_WG * k candidates sorted, the best k out.
__global__ __launch_bounds__(256) void k_topk_final(const float *__restrict__ cv, const int *__restrict__ ci, int nc,
                                                    int k, float *__restrict__ out_v, int32_t *__restrict__ out_i) {
    constexpr int N = TOPK_WG * TOPK_MAX;
    __shared__ float v[N];
    __shared__ int ix[N];
    const int64_t o = (int64_t)blockIdx.x * nc;
    for (int t = threadIdx.x; t < N; t += 256) {
        v[t] = t < nc ? cv[o + t] : -INFINITY;
        ix[t] = t < nc ? ci[o + t] : INT_MAX;
    }
    bitonic<N>(v, ix);
    for (int t = threadIdx.x; t < k; t += 256) {
        out_v[(int64_t)blockIdx.x * k + t] = v[t];
        out_i[(int64_t)blockIdx.x * k + t] = ix[t];
    }
}

// ---------------------------------------------------------------------------
size_t argmax_scratch_bytes(int rows) { return (size_t)rows * ARGMAX_WG * 8; }

hipError_t launch_argmax(const float *x, int n, int rows, void *scratch, int32_t *out, int32_t *seq, int32_t *pos,
                         hipStream_t s) {
    float *pv = (float *)scratch;
    int *pi = (int *)((char *)scratch + (size_t)rows * ARGMAX_WG * 4);
    hipLaunchKernelGGL(k_argmax_part, dim3(ARGMAX_WG, rows), dim3(256), 0, s, x, n, pv, pi);
    hipLaunchKernelGGL(k_argmax_final, dim3(rows), dim3(256), 0, s, pv, pi, ARGMAX_WG, out, seq, pos);
    return hipGetLastError();
}

__global__ void k_advance(int32_t *pos) { *pos += 1; }
__global__ void k_set_pos(int32_t *pos, int32_t v) { *pos = v; }

hipError_t launch_advance(int32_t *pos, hipStream_t s) {
    hipLaunchKernelGGL(k_advance, dim3(1), dim3(1), 0, s, pos);
    return hipGetLastError();
}

hipError_t launch_set_pos(int32_t *pos, int32_t v, hipStream_t s) {
    hipLaunchKernelGGL(k_set_pos, dim3(1), dim3(1), 0, s, pos, v);
    return hipGetLastError();
}

size_t topk_scratch_bytes(int rows) { return (size_t)rows * TOPK_WG * TOPK_MAX * 8; }
int topk_max() { return TOPK_MAX; }
int topk_max_n() { return TOPK_WG * TOPK_SLICE; }

hipError_t launch_topk(const float *x, int n, int k, int rows, void *scratch, float *vals, int32_t *ids,
                       hipStream_t s) {
    if (rows < 1 || k < 1 || k > TOPK_MAX || n > TOPK_WG * TOPK_SLICE) return hipErrorInvalidValue;
    float *cv = (float *)scratch;
    int *ci = (int *)((char *)scratch + (size_t)rows * TOPK_WG * TOPK_MAX * 4);
    hipLaunchKernelGGL(k_topk_part, dim3(TOPK_WG, rows), dim3(256), 0, s, x, n, k, cv, ci);
    hipLaunchKernelGGL(k_topk_final, dim3(rows), dim3(256), 0, s, cv, ci, TOPK_WG * k, k, vals, ids);
    return hipGetLastError();
}

}  // namespace ts5hip
