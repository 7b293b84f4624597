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
// Top-k (k <= 64) in two launches, each an exact selection then a small sort:
//  1. one workgroup per 1024-logit slice of a row finds the key of its k-th
//     best logit by a 4-pass, 8-bit radix select over order-preserving keys
//     of the values, gathers the logits at or above it and sorts them (rank
//     order: larger value, then smaller id); its best k go out;
//  2. one workgroup per row gathers the entries of the slices' lists at or
//     above a bound on the row's k-th best and sorts them: the row's best k
//     are among them (a slice holds at most k of them).
// Logits equal to the k-th best are all gathered and the sort orders them by
// id; past TOPK_CAND of them (a row of many equal logits) the slices' sorted
// lists are merged instead, a head at a time. NaN logits rank below every
// number (their keys are the lowest).
// ---------------------------------------------------------------------------
constexpr int TOPK_SLICE = 1024, TOPK_NWG = 256, TOPK_MAX = 64, TOPK_CAND = 1024;

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

// Larger value -> larger key; -0 and +0 one key (they rank by id, as equal
// values do); NaN -> 0.
__device__ inline uint32_t order_key(float f) {
    if (f != f) return 0u;
    const uint32_t u = f == 0.f ? 0u : __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

struct TopkLds {
    int hist[256];
    int bin, above, count;
    float v[TOPK_CAND];
    int ix[TOPK_CAND];
    float bv[4];
    int bi[4];
};

// The key of the k-th largest of the keys the workgroup's 256 threads hold
// (M a thread, `valid` of them used): every key above it counts < k, at or
// above >= k.
template <int M>
__device__ inline uint32_t radix_kth(const uint32_t (&key)[M], int valid, int k, TopkLds &S) {
    const int t = threadIdx.x, lane = t & 63;
    uint32_t prefix = 0, mask = 0;
    int want = k;
    for (int shift = 24; shift >= 0; shift -= 8) {
        S.hist[t] = 0;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < M; j++)
            if (j < valid && (key[j] & mask) == prefix) atomicAdd(&S.hist[(key[j] >> shift) & 255], 1);
        __syncthreads();
        if (t < 64) {
            // Lane i holds bins 255 - 4i .. 252 - 4i (high bins first).
            int c[4], tot = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) c[q] = S.hist[255 - 4 * lane - q], tot += c[q];
            int incl = tot;  // inclusive prefix over lanes 0..lane
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y = __shfl_up(incl, o, 64);
                if (lane >= o) incl += y;
            }
            int run = incl - tot;  // keys in higher bins than this lane's
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if (run < want && run + c[q] >= want) S.bin = 255 - 4 * lane - q, S.above = run;
                run += c[q];
            }
        }
        __syncthreads();
        want -= S.above;
        prefix |= (uint32_t)S.bin << shift;
        mask |= 255u << shift;
        __syncthreads();
    }
    return prefix;
}

// The entries whose key is at or above kth into S.v / S.ix (count in
// S.count; those past TOPK_CAND are counted, not stored).
template <int M>
__device__ inline void gather_at_or_above(const uint32_t (&key)[M], const float (&val)[M], const int (&id)[M],
                                          int valid, uint32_t kth, TopkLds &S) {
    if (threadIdx.x == 0) S.count = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < M; j++) {
        if (j < valid && key[j] >= kth) {
            const int at = atomicAdd(&S.count, 1);
            if (at < TOPK_CAND) S.v[at] = val[j], S.ix[at] = id[j];
        }
    }
    __syncthreads();
}

// Sorts S.v[0 .. total) (total <= TOPK_CAND) into rank order.
__device__ inline void sort_gathered(int total, TopkLds &S) {
    const int nsort = total <= 64 ? 64 : total <= 128 ? 128 : total <= 256 ? 256 : total <= 512 ? 512 : 1024;
    for (int j = total + (int)threadIdx.x; j < nsort; j += 256) S.v[j] = -INFINITY, S.ix[j] = INT_MAX;
    switch (nsort) {
    case 64: bitonic<64>(S.v, S.ix); break;
    case 128: bitonic<128>(S.v, S.ix); break;
    case 256: bitonic<256>(S.v, S.ix); break;
    case 512: bitonic<512>(S.v, S.ix); break;
    default: bitonic<TOPK_CAND>(S.v, S.ix); break;
    }
}

// grid (nwg, rows): workgroup x of row y over logits [1024 x, 1024 (x + 1)).
__global__ __launch_bounds__(256) void k_topk_part(const float *__restrict__ x, int n, int k, float *__restrict__ cv,
                                                   int *__restrict__ ci) {
    __shared__ TopkLds S;
    const float *xr = x + (int64_t)blockIdx.y * n;
    const int lo = blockIdx.x * TOPK_SLICE;
    constexpr int M = TOPK_SLICE / 256;
    uint32_t key[M];
    float val[M];
    int id[M];
#pragma unroll
    for (int j = 0; j < M; j++) {
        const int g = lo + threadIdx.x + 256 * j;
        val[j] = g < n ? xr[g] : -INFINITY;
        id[j] = g < n ? g : INT_MAX;
        key[j] = g < n ? order_key(val[j]) : 0u;
    }
    const int have = min(TOPK_SLICE, n - lo);  // > 0
    const int kk = min(k, have);
    const uint32_t kth = radix_kth<M>(key, M, kk, S);
    gather_at_or_above<M>(key, val, id, M, kth, S);
    const int total = S.count;
    const int64_t o = ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * k;
    if (total <= TOPK_CAND) {
        sort_gathered(total, S);
        for (int t = threadIdx.x; t < k; t += 256) cv[o + t] = S.v[t], ci[o + t] = S.ix[t];  // past have: padding
        return;
    }
    // Many equal logits: a full sort of the slice.
    for (int j = 0; j < M; j++) S.v[threadIdx.x + 256 * j] = val[j], S.ix[threadIdx.x + 256 * j] = id[j];
    bitonic<TOPK_SLICE>(S.v, S.ix);
    for (int t = threadIdx.x; t < k; t += 256) cv[o + t] = S.v[t], ci[o + t] = S.ix[t];
}

// One workgroup per row over its nwg lists of k (each in rank order).
// A bound first: with j = ceil(k / nwg) and m = ceil(k / j), the m-th best
// of the lists' j-th entries, T, has m lists holding j entries each at or
// above it, so at least k do; the entries at or above T (for unsorted logits
// a few more than k) are gathered and sorted.
__global__ __launch_bounds__(256) void k_topk_final(const float *__restrict__ cv, const int *__restrict__ ci, int nwg,
                                                    int k, float *__restrict__ out_v, int32_t *__restrict__ out_i) {
    __shared__ TopkLds S;
    const int t = threadIdx.x;
    const float *lv = cv + ((int64_t)blockIdx.x * nwg + t) * k;
    const int *li = ci + ((int64_t)blockIdx.x * nwg + t) * k;
    const int j = (k + nwg - 1) / nwg, m = (k + j - 1) / j;
    uint32_t jk[1] = {0u};
    if (t < nwg && li[j - 1] != INT_MAX) jk[0] = order_key(lv[j - 1]);
    const uint32_t T = radix_kth<1>(jk, 1, m, S);
    // This list's entries at or above T: a prefix of it.
    if (t == 0) S.count = 0;
    __syncthreads();
    if (t < nwg) {
        for (int e = 0; e < k; e++) {
            if (li[e] == INT_MAX || order_key(lv[e]) < T) break;
            const int at = atomicAdd(&S.count, 1);
            if (at < TOPK_CAND) S.v[at] = lv[e], S.ix[at] = li[e];
        }
    }
    __syncthreads();
    const int total = S.count;
    float *ov = out_v + (int64_t)blockIdx.x * k;
    int32_t *oi = out_i + (int64_t)blockIdx.x * k;
    if (total <= TOPK_CAND) {
        sort_gathered(total, S);
        for (int e = t; e < k; e += 256) ov[e] = S.v[e], oi[e] = S.ix[e];
        return;
    }
    // Many equal logits: merge the sorted lists, the best head k times.
    int head = 0;
    for (int e = 0; e < k; e++) {
        float hv = -INFINITY;
        int hi = INT_MAX;
        if (t < nwg && head < k) hv = lv[head], hi = li[head];
        float wv = hv;
        int wi = hi;
        block_best(wv, wi, S.bv, S.bi);
        if (t == 0) S.bv[0] = wv, S.bi[0] = wi, ov[e] = wv, oi[e] = wi;
        __syncthreads();
        if (t < nwg && head < k && hi == S.bi[0] && hv == S.bv[0] && hi != INT_MAX) head++;  // ids are unique
        __syncthreads();
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

size_t topk_scratch_bytes(int rows) { return (size_t)rows * TOPK_NWG * TOPK_MAX * 8; }
int topk_max() { return TOPK_MAX; }
int topk_max_n() { return TOPK_NWG * TOPK_SLICE; }

hipError_t launch_topk(const float *x, int n, int k, int rows, void *scratch, float *vals, int32_t *ids,
                       hipStream_t s) {
    if (rows < 1 || k < 1 || k > TOPK_MAX || n < 1 || n > TOPK_NWG * TOPK_SLICE) return hipErrorInvalidValue;
    const int nwg = (n + TOPK_SLICE - 1) / TOPK_SLICE;
    float *cv = (float *)scratch;
    int *ci = (int *)((char *)scratch + (size_t)rows * TOPK_NWG * TOPK_MAX * 4);
    hipLaunchKernelGGL(k_topk_part, dim3(nwg, rows), dim3(256), 0, s, x, n, k, cv, ci);
    hipLaunchKernelGGL(k_topk_final, dim3(rows), dim3(256), 0, s, cv, ci, nwg, k, vals, ids);
    return hipGetLastError();
}

}  // namespace ts5hip
