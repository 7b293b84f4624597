// One-token Q4_K matvecs over row-packed steps (mv_run's BR = 4): each
// 16-lane row of a wave on its own matrix row, 4 blocks a step, so rows of
// 12 or 20 blocks (3072 and 5120 wide) keep every lane busy where whole
// 16-block steps would leave most of a row's last step empty. Launched by
// matvec.hip's dispatch; a file of their own, so that the code of the other
// matvec kernels keeps its place.
#include <climits>

#include "kernels.h"
#include "mv_core.h"

namespace ts5hip {

// Arguments as k_mv's (the leading ones preloaded into SGPRs); no pick.
template <int MODE, int RUNS, bool NORM>
__global__ __launch_bounds__(4 * WAVE) void k_mv_packed(const void *w, const void *w2, const float *x,
                                                        const float *norm_w, float *y, int nrows, int n_in, int nwg,
                                                        float eps, MvTail tail) {
    static_assert(MODE != MV_ARGMAX, "no pick on row-packed steps");
    MvArgs a;
    a.t = tail.t, a.w = w, a.w2 = w2, a.nrows = nrows, a.nb = n_in / Q4K::VALUES, a.n_in = n_in, a.x = x;
    a.norm_w = norm_w, a.eps = eps, a.y = y, a.y_in = tail.y_in;
    a.nfirst = tail.nfirst, a.n1 = tail.n1, a.gelu = tail.gelu;
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[2 * 4];
    float best_v;
    int best_i;
    auto fetch_tail = [&]() {
        if constexpr (MODE == MV_ADD) asm volatile("" ::"s"(a.y_in));
    };
    mv_run<Q4K, 1, 4, 1, MODE, RUNS, NORM, 4>(a, blockIdx.x, nwg, lds, red, fetch_tail, best_v, best_i);
}

hipError_t launch_mv_packed(int mode, int runs, bool norm, dim3 g, dim3 b, size_t lds, hipStream_t s, const void *w,
                            const void *w2, const float *x, const float *norm_w, float *y, int nrows, int n_in,
                            int nwg, float eps, const MvTail &tail) {
    auto go = [&](auto mc) {
        constexpr int MD = decltype(mc)::value;
#define TS5_MVP(RUNS, NORM) \
    hipLaunchKernelGGL((k_mv_packed<MD, RUNS, NORM>), g, b, lds, s, w, w2, x, norm_w, y, nrows, n_in, nwg, eps, tail)
        if (runs == 1 && norm) TS5_MVP(1, true);
        else if (runs == 1) TS5_MVP(1, false);
        else if (runs == 2 && norm) TS5_MVP(2, true);
        else if (runs == 2) TS5_MVP(2, false);
        else if (runs == 4) TS5_MVP(4, false);
        else TS5_MVP(0, false);
#undef TS5_MVP
    };
    if (mode == MV_STORE) go(std::integral_constant<int, MV_STORE>{});
    else if (mode == MV_ADD) go(std::integral_constant<int, MV_ADD>{});
    else if (mode == MV_GLU) go(std::integral_constant<int, MV_GLU>{});
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace ts5hip
