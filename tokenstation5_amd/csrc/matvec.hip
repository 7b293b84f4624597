// One-token k-quant matvec kernels (plain, accumulating into a residual,
// fused gate/up + SiLU, and the output head with the greedy argmax) over the
// device core in mv_core.h.
#include <algorithm>
#include <climits>

#include "kernels.h"
#include "mv_core.h"

namespace ts5hip {

// The arguments every mode needs come first and one by one: 14 dwords the
// command processor preloads into SGPRs at wave launch (the matvec file builds
// with -amdgpu-kernarg-preload-count=16; two of the 16 user SGPRs hold the
// argument pointer), so a launch does not start with a round trip to its
// argument buffer. nwg is the grid size.
template <class F, int R, int WAVES, int KS, int MODE, int RUNS, bool NORM>
__global__ __launch_bounds__(WAVES *WAVE) void k_mv(const void *w, const void *w2, const float *x,
                                                    const float *norm_w, float *y, int nrows, int n_in, int nwg,
                                                    float eps, MvTail tail) {
    MvArgs a;
    a.t = tail.t, a.w = w, a.w2 = w2, a.nrows = nrows, a.nb = tail.nb, a.n_in = n_in, a.x = x, a.norm_w = norm_w;
    a.eps = eps, a.y = y, a.y_in = tail.y_in;
    a.best_v = tail.best_v, a.best_i = tail.best_i, a.counter = tail.counter, a.out = tail.out, a.seq = tail.seq;
    a.pos = tail.pos;
    a.nfirst = tail.nfirst, a.n1 = tail.n1, a.gelu = tail.gelu;
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[2 * WAVES];
    __shared__ int last;
    float best_v;
    int best_i;
    // The type and block count are compile-time facts of F and n_in; only the
    // residual pointer of MV_ADD is fetched, once the first loads are out.
    a.nb = n_in / F::VALUES;
    auto fetch_tail = [&]() {
        if constexpr (MODE == MV_ADD) asm volatile("" ::"s"(a.y_in));
    };
    mv_run<F, R, WAVES, KS, MODE, RUNS, NORM>(a, blockIdx.x, nwg, lds, red, fetch_tail, best_v, best_i);
    if (MODE != MV_ARGMAX) return;
    // Each workgroup's best, then the last workgroup to finish picks the
    // winner. Workgroup w counts into sub-counter w % ARGMAX_FAN, the last
    // arrival there (which zeroes it) into the top counter a.counter[0].
    if (threadIdx.x == 0) {
        st_dev(a.best_v + blockIdx.x, best_v);
        st_dev(a.best_i + blockIdx.x, best_i);
        wait_stores();
        const int n = (int)gridDim.x, sub = blockIdx.x % ARGMAX_FAN;
        int *sc = a.counter + CTR_STRIDE * (1 + sub);
        last = 0;
        if (atomicAdd(sc, 1) == (n - sub + ARGMAX_FAN - 1) / ARGMAX_FAN - 1) {
            st_dev(sc, 0);
            last = atomicAdd(a.counter, 1) == min(n, ARGMAX_FAN) - 1;
        }
    }
    __syncthreads();
    if (!last) return;
    best_v = -INFINITY, best_i = INT_MAX;
    for (int k = threadIdx.x; k < (int)gridDim.x; k += WAVES * WAVE) {
        const float v = a.best_v[k];
        const int i = a.best_i[k];
        if (v > best_v || (v == best_v && i < best_i)) best_v = v, best_i = i;
    }
    best_pick_wave(best_v, best_i);
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[wave] = best_v, red[WAVES + wave] = __int_as_float(best_i);
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < WAVES; k++) {
            const float v = red[k];
            const int i = __float_as_int(red[WAVES + k]);
            if (v > best_v || (v == best_v && i < best_i)) best_v = v, best_i = i;
        }
        if (best_i == INT_MAX) best_i = 0;  // every logit NaN
        a.out[0] = best_i;
        if (a.seq) {
            const int p = *a.pos;
            a.seq[p + 1] = best_i;
            *a.pos = p + 1;
        }
        st_dev(a.counter, 0);  // ready for the next launch (graph replays)
    }
}

// ---------------------------------------------------------------------------
// Launch shapes. Rows per group = R * WAVES; the grid is capped at two
// workgroups per CU, so large matrices loop over their groups with the next
// step's weights in flight.
// ---------------------------------------------------------------------------
constexpr double MV_FIRST_SHARE = 0.62;  // row groups of the workgroups dispatched first (one a CU)
constexpr int MV_WG_PER_CU = 2;
constexpr int MV_GLU_WAVES = 4;
constexpr int MV_GLU_R = 1;  // with its alternating buffers, 16.3 us on the 8B gate/up against 16.8 at 2 rows
constexpr int MV_Q6_R = 2;   // the 8B head: 97 against 107 us at 4 rows a wave
constexpr int MV_R = 4;      // rows a wave of a persistent Q4_K grid
static int g_n_cu = 256;
void set_cu_count(int n) { g_n_cu = n > 0 ? n : 256; }
// The grid cap, and so the most per-workgroup (value, row) pairs of the
// head's argmax.
static size_t mv_max_grid() { return (size_t)MV_WG_PER_CU * g_n_cu; }

template <class F, int R, int WAVES, int KS, int MODE, int BR = 0>
static hipError_t mv_go(const MvArgs &a, hipStream_t s) {
    if (a.nrows > INT32_MAX) return hipErrorInvalidValue;  // the kernel takes a 32-bit row count
    constexpr int BPI = WAVE / F::LPB, LR = BR ? BPI / BR : 1;  // rows a row-packed slot spans
    const int64_t rpg = (int64_t)R * LR * (WAVES / KS);
    const int64_t ngroups = (a.nrows + rpg - 1) / rpg;
    const int64_t cap = (int64_t)mv_max_grid();
    const int64_t per = (ngroups + cap - 1) / cap;  // groups per workgroup
    // Past the cap every CU holds two workgroups, which the first-dispatched
    // share below assumes. (A grid of ceil(groups / per) left some CUs one
    // workgroup: 608 groups gave 304 workgroups, the first 256 one group each
    // and the other 48 seven or eight; the draft's 896 x 4864 gate/up took
    // 10.9 us instead of 6.)
    const unsigned grid = (unsigned)std::min(ngroups, cap);
    // The prologue's inputs in registers (runs per thread, norm weights) when
    // they fit: up to 2 runs with the norm, 4 without; else the two-pass one.
    const int nr = a.n_in / 16, nt = WAVES * WAVE;
    const bool norm = a.norm_w != nullptr;
    const dim3 g(grid), b(WAVES * WAVE);
    const size_t lds = act_bytes(a.n_in);
    // A persistent grid of two workgroups a CU: the ones dispatched first
    // (one a CU) run ahead of the second on the same CU (their waves are
    // older), so they take a larger share of the groups and both halves end
    // together (with equal shares the gate/up's second half ended 4 us after
    // the first; at 62 % the halves end within 0.4 us: 17.0 -> 16.1 us, the
    // Q6_K head 100.8 -> 97 us).
    int nfirst = 0, n1 = 0;
    if (per > 1 && grid > (unsigned)g_n_cu) {
        nfirst = g_n_cu;
        const int64_t want = (int64_t)(MV_FIRST_SHARE * (double)ngroups / nfirst + 0.5) * nfirst;
        n1 = (int)std::min<int64_t>(std::max<int64_t>(want, nfirst), ngroups - ((int64_t)grid - nfirst));
    }
    const MvTail tail{a.t, a.nb, nfirst, n1, a.y_in, a.best_v, a.best_i, a.counter, a.out, a.seq, a.pos, a.gelu};
    if constexpr (BR != 0) {  // row-packed steps (matvec_packed.hip)
        static_assert(std::is_same_v<F, Q4K> && R == 1 && WAVES == 4 && KS == 1 && BR == 4, "the packed kernels built");
        const int runs = nr <= nt ? 1 : nr <= 2 * nt ? 2 : nr <= 4 * nt && !norm ? 4 : 0;
        return launch_mv_packed(MODE, runs, norm && runs > 0 && runs <= 2, g, b, lds, s, a.w, a.w2, a.x, a.norm_w,
                                a.y, (int)a.nrows, a.n_in, (int)grid, a.eps, tail);
    }
#define TS5_MV_LAUNCH(RUNS, NORM)                                                                                 \
    hipLaunchKernelGGL((k_mv<F, R, WAVES, KS, MODE, RUNS, NORM>), g, b, lds, s, a.w, a.w2, a.x, a.norm_w, a.y,        \
                       (int)a.nrows, a.n_in, (int)grid, a.eps, tail)
    if constexpr (BR == 0) {
        if (nr <= nt && norm) TS5_MV_LAUNCH(1, true);
        else if (nr <= nt) TS5_MV_LAUNCH(1, false);
        else if (nr <= 2 * nt && norm) TS5_MV_LAUNCH(2, true);
        else if (nr <= 2 * nt) TS5_MV_LAUNCH(2, false);
        else if (nr <= 4 * nt && !norm) TS5_MV_LAUNCH(4, false);
        else TS5_MV_LAUNCH(0, false);
    }
#undef TS5_MV_LAUNCH
    return hipGetLastError();
}

// Q4_K rows of more than one step (nb > 16 blocks, the down projection):
// the workgroup's waves split each row's blocks, so that a CU has more weight
// bytes in flight than its few row groups give it.
constexpr int MV_KS = 2;         // block splits of a row (4 measured slower)
constexpr int MV_KS_R = 4;
constexpr int MV_KS_WAVES = 8;   // 16 waves spill
constexpr int MV_KS_MINNB = 17;  // rows of more than one 16-block step

// Rows per wave of a Q4_K matvec whose row groups all fit the grid at once
// (one step each): the count that leaves the busiest CU the fewest rows per
// wave, ties to more rows per wave (more bytes in flight). QKV of the 8B
// (6144 rows): 3 rows, 512 workgroups, two a CU (7.6 -> 6.8 us); at 4 rows
// its 384 workgroups leave half the CUs with two and half with one.
static int mv_rows_per_wave(int64_t nrows) {
    if ((nrows + 15) / 16 > (int64_t)mv_max_grid()) return MV_R;  // a persistent grid
    int best = 4;
    int64_t best_cost = INT64_MAX;
    for (int r = 4; r >= 2; r--) {
        const int64_t groups = (nrows + 4 * r - 1) / (4 * r);
        const int64_t cost = (groups + g_n_cu - 1) / g_n_cu * r;
        if (cost < best_cost) best = r, best_cost = cost;
    }
    return best;
}

template <int MODE>
static hipError_t mv_dispatch(const MvArgs &a, hipStream_t s) {
    // Q4_K rows of 4n blocks short of a whole 16-block step (3072 and 5120
    // wide: 12 and 20 blocks) on row-packed steps of 4 blocks, every lane busy.
    const bool packed = a.t == T_Q4_K && MODE != MV_ARGMAX && a.nb % 16 != 0 && a.nb % 4 == 0 && a.nb < 32;
    if constexpr (MODE != MV_ARGMAX)
        if (packed) return mv_go<Q4K, 1, 4, 1, MODE, 4>(a, s);
    if constexpr (MODE == MV_GLU) {
        switch (a.t) {
        case T_Q4_K: return mv_go<Q4K, MV_GLU_R, MV_GLU_WAVES, 1, MODE>(a, s);
        case T_Q6_K: return mv_go<Q6K, 2, 4, 1, MODE>(a, s);
        case T_Q8_0: return mv_go<Q80, 1, 4, 1, MODE>(a, s);  // the draft's 896 x 4864: 0.794 -> 0.790 ms a token at 1 row
        case T_Q8SM: return mv_go<Q8M, 2, 4, 1, MODE>(a, s);
        case T_F16: return mv_go<F16W, 2, 4, 1, MODE>(a, s);
        case T_F32: return mv_go<F32W, 2, 4, 1, MODE>(a, s);
        }
    } else {
        switch (a.t) {
        case T_Q4_K:
            if (MODE != MV_ARGMAX && a.nb >= MV_KS_MINNB) {
                // Too few rows for a group a CU at 4 rows a wave (the draft's
                // 896-row down: 56 groups), or a count that leaves CUs with one
                // group and others two (the 48x5120 target's 5120-row down: 320
                // groups): one row a wave, 4 times the groups (a draft token
                // 0.843 -> 0.796 ms with the Q8_0 rule below; the target's
                // token 289 -> 310 tok/s).
                const int64_t g4 = (a.nrows + MV_KS_R * 4 - 1) / (MV_KS_R * 4);
                if (g4 < g_n_cu || (g4 < 2 * g_n_cu && g4 % g_n_cu != 0))
                    return mv_go<Q4K, 1, MV_KS_WAVES, MV_KS, MODE>(a, s);
                return mv_go<Q4K, MV_KS_R, MV_KS_WAVES, MV_KS, MODE>(a, s);
            }
            switch (mv_rows_per_wave(a.nrows)) {
            case 3: return mv_go<Q4K, 3, 4, 1, MODE>(a, s);
            case 2: return mv_go<Q4K, 2, 4, 1, MODE>(a, s);
            default: return mv_go<Q4K, 4, 4, 1, MODE>(a, s);
            }
        case T_Q6_K: return mv_go<Q6K, MV_Q6_R, 4, 1, MODE>(a, s);
        case T_Q8_0:  // one row a wave where 4 leave CUs without a group (the draft's 896-1152 rows)
            if (MODE != MV_ARGMAX && (a.nrows + 15) / 16 < g_n_cu) return mv_go<Q80, 1, 4, 1, MODE>(a, s);
            return mv_go<Q80, 4, 4, 1, MODE>(a, s);
        case T_Q8SM: return mv_go<Q8M, 4, 4, 1, MODE>(a, s);
        case T_F16: return mv_go<F16W, 4, 4, 1, MODE>(a, s);
        case T_F32: return mv_go<F32W, 2, 4, 1, MODE>(a, s);
        }
    }
    return hipErrorInvalidValue;
}

static MvArgs mv_args(uint32_t t, const void *w, int64_t ne0, int64_t ne1, const float *x, const float *norm_w,
                      float eps, float *y) {
    MvArgs a{};
    const int bv = t == T_F16 || t == T_F32 ? 32 : block_values(t);  // float rows: 32-value blocks
    a.t = t, a.w = w, a.w2 = nullptr, a.nrows = ne1, a.nb = (int)(ne0 / bv), a.n_in = (int)ne0;
    a.x = x, a.norm_w = norm_w, a.eps = eps, a.y = y, a.y_in = y;
    return a;
}

hipError_t launch_matvec(uint32_t t, const void *w, int64_t ne0, int64_t ne1, const float *x, const float *norm_w,
                         float eps, float *y, int add, hipStream_t s) {
    const MvArgs a = mv_args(t, w, ne0, ne1, x, norm_w, eps, y);
    return add ? mv_dispatch<MV_ADD>(a, s) : mv_dispatch<MV_STORE>(a, s);
}

hipError_t launch_matvec_glu(uint32_t t, const void *wg, const void *wu, int64_t ne0, int64_t ne1, const float *x,
                             const float *norm_w, float eps, float *y, hipStream_t s, int gelu) {
    MvArgs a = mv_args(t, wg, ne0, ne1, x, norm_w, eps, y);
    a.w2 = wu;
    a.gelu = gelu ? 1 : 0;
    return mv_dispatch<MV_GLU>(a, s);
}

// Several tokens of F16 / F32 rows (no matrix-core path): the one-token
// matvec per token.
hipError_t launch_matvec_tokens(uint32_t t, const void *w, const void *w2, int64_t ne0, int64_t ne1, const float *x,
                                int64_t xstride, const float *norm_w, float eps, int ntok, int mode, float *y,
                                int64_t ldy, hipStream_t s) {
    for (int k = 0; k < ntok; k++) {
        const float *xk = x + (int64_t)k * xstride;
        float *yk = y + (int64_t)k * ldy;
        const int m = mode & ~GLU_GELU;
        const hipError_t e = m == 2 ? launch_matvec_glu(t, w, w2, ne0, ne1, xk, norm_w, eps, yk, s, mode & GLU_GELU)
                                    : launch_matvec(t, w, ne0, ne1, xk, norm_w, eps, yk, m == 1, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Per-workgroup partials of the argmax epilogue: best values then best rows.
size_t matvec_argmax_scratch_bytes() { return 8 * mv_max_grid(); }

hipError_t launch_matvec_argmax(uint32_t t, const void *w, int64_t ne0, int64_t ne1, const float *x,
                                const float *norm_w, float eps, float *y, void *scratch, int *counter, int32_t *out,
                                int32_t *seq, int32_t *pos, hipStream_t s) {
    MvArgs a = mv_args(t, w, ne0, ne1, x, norm_w, eps, y);
    a.counter = counter;
    a.best_v = (float *)scratch;
    a.best_i = (int *)((uint8_t *)scratch + 4 * mv_max_grid());
    a.out = out, a.seq = seq, a.pos = pos;
    return mv_dispatch<MV_ARGMAX>(a, s);
}

}  // namespace ts5hip
