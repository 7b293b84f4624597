// Decode attention of one query per cache at head dimension 128 with its key
// loop on the matrix cores (attn_m1.h), launched by launch_attn (attention.hip)
// for caches past the LDS kernel's reach and batches of queries on caches of
// their own. A file of its own, so that the code of the decode kernels
// around it keeps its place.
#include "attn_m1.h"

namespace ts5hip {

// flags: 1 kv_per_batch, 2 append, 4 rope; the leading scalar arguments are
// preloaded into SGPRs at wave launch (built with the kernarg preload count).
template <int G, bool F16>
__global__ __launch_bounds__(M1_NT) void k_attn_m1(const int8_t *k8, const uint16_t *ks, const int8_t *v8,
                                                   const uint16_t *vs, const int32_t *n_keys, int n_ctx, int HKV,
                                                   int flags, int n_split, AttnArgs tail) {
    __shared__ M1Lds<G> S;
    AttnArgs a = tail;
    a.kv = KvLayer{const_cast<int8_t *>(k8), const_cast<uint16_t *>(ks), const_cast<int8_t *>(v8),
                   const_cast<uint16_t *>(vs)};
    a.n_keys = n_keys, a.n_ctx = n_ctx, a.HKV = HKV;
    a.kv_per_batch = flags & 1, a.append = (flags >> 1) & 1, a.rope = (flags >> 2) & 1;
    attn_m1<G, F16>(a, blockIdx.x, blockIdx.y, blockIdx.z, n_split, S);
}

hipError_t launch_attn_m1(int G, bool f16, dim3 grid, const AttnArgs &a, hipStream_t s) {
    const int flags = (a.kv_per_batch ? 1 : 0) | (a.append ? 2 : 0) | (a.rope ? 4 : 0);
    auto go = [&](auto gc, auto fc) {
        constexpr int GG = decltype(gc)::value;
        constexpr bool FF = decltype(fc)::value;
        hipLaunchKernelGGL((k_attn_m1<GG, FF>), grid, dim3(M1_NT), 0, s, (const int8_t *)a.kv.k,
                           (const uint16_t *)a.kv.ks, (const int8_t *)a.kv.v, (const uint16_t *)a.kv.vs, a.n_keys,
                           a.n_ctx, a.HKV, flags, (int)grid.x, a);
    };
    auto by_g = [&](auto fc) {
        switch (G) {
        case 1: go(std::integral_constant<int, 1>{}, fc); return hipSuccess;
        case 2: go(std::integral_constant<int, 2>{}, fc); return hipSuccess;
        case 4: go(std::integral_constant<int, 4>{}, fc); return hipSuccess;
        case 5: go(std::integral_constant<int, 5>{}, fc); return hipSuccess;
        case 7: go(std::integral_constant<int, 7>{}, fc); return hipSuccess;
        case 8: go(std::integral_constant<int, 8>{}, fc); return hipSuccess;
        default: return hipErrorInvalidValue;
        }
    };
    const hipError_t e = f16 ? by_g(std::true_type{}) : by_g(std::false_type{});
    return e != hipSuccess ? e : hipGetLastError();
}

}  // namespace ts5hip
