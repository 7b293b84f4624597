// One decode token as one persistent kernel: every workgroup stays resident
// for the whole token and the phases of each layer are separated by grid
// barriers instead of kernel boundaries (a kernel boundary costs ~4 us on
// this GPU; a token of the 8B has ~160 phase changes).
//
// Phases of a token at position p (state[0]):
//   embed            x = row seq[p] of token_embd (each workgroup a slice)
//   per layer        QKV matvec (rmsnorm fused)  | attention (RoPE, q8 append,
//                    split-K, last-workgroup merge) | O matvec (x +=) |
//                    gate/up + SiLU (rmsnorm fused) | down matvec (x +=)
//   head             logits = W_out rmsnorm(x) [+ greedy argmax -> seq[p+1]]
//   then state[0] = p + 1.
// Each matvec phase issues its first weight loads before waiting at the
// barrier that precedes it, so HBM keeps streaming across phase changes.
//
// Termination: the grid is launched cooperatively (every workgroup
// resident). A barrier that waits longer than a bounded spin count sets an
// error flag and returns; every later barrier then returns at once, so the
// kernel always exits and the host reports the error.
#include <cstring>

#include "attn_core.h"
#include "kernels.h"
#include "mv_core.h"

namespace ts5hip {

// Barrier state: a global count and generation, and per group of GROUP
// workgroups a count and generation on lines of their own.
constexpr int BAR_GROUP = 32, BAR_MAX_GROUPS = 64;
struct GridBar {
    unsigned count, gen;
    int err;
    unsigned pad[29];
    unsigned gcount[BAR_MAX_GROUPS][32];  // one 128-byte line per group
    unsigned ggen[BAR_MAX_GROUPS][32];
};

constexpr unsigned BAR_SPIN_LIMIT = 1u << 22;  // ~seconds of waiting

__device__ inline unsigned ld_rlx(unsigned *p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline unsigned add_rlx(unsigned *p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline unsigned xchg_rlx(unsigned *p, unsigned v) {
    return __hip_atomic_exchange(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_rlx(unsigned *p, unsigned v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// Spins until *p != v; false (and the error flag set) after the spin limit.
__device__ inline bool wait_change(GridBar *bar, unsigned *p, unsigned v) {
    unsigned spins = 0;
    while (ld_rlx(p) == v) {
        __builtin_amdgcn_s_sleep(1);
        if (++spins > BAR_SPIN_LIMIT) {
            __hip_atomic_store(&bar->err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
    }
    return true;
}

// Every workgroup of the grid arrives (its stores performed) before any leaves.
// Two levels, relaxed device-scope atomics only: a workgroup counts on its
// group's line; the group's last arriver counts on the global line and, once
// the whole grid is in, bumps the group's generation, which the group's
// members poll. 512 arrivals on one line would serialise at the atomic unit
// (~9 us measured on the full grid; ~3 us this way). The data handoff is by
// coherent stores into buffers no reader has cached (common.h), so there is
// no cache maintenance. A count is reset before the generation that releases
// the waiters is published: the generation stored depends on the exchange's
// result, so it cannot be issued first.
__device__ inline void grid_barrier(GridBar *bar, unsigned nwg, int *lds_flag) {
    wait_stores();
    __syncthreads();
    if (threadIdx.x == 0) {
        const int err = __hip_atomic_load(&bar->err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (!err) {
            const unsigned grp = blockIdx.x / BAR_GROUP, ngrp = (nwg + BAR_GROUP - 1) / BAR_GROUP;
            const unsigned gsize = min((unsigned)BAR_GROUP, nwg - grp * BAR_GROUP);
            unsigned *gc = &bar->gcount[grp][0], *gg = &bar->ggen[grp][0];
            const unsigned ggv = ld_rlx(gg);
            if (add_rlx(gc, 1u) == gsize - 1) {
                const unsigned g = ld_rlx(&bar->gen);
                const unsigned o1 = xchg_rlx(gc, 0u);
                if (add_rlx(&bar->count, 1u + (o1 == 0xffffffffu ? 1u : 0u)) == ngrp - 1) {
                    const unsigned o = xchg_rlx(&bar->count, 0u);
                    st_rlx(&bar->gen, g + 1 + (o == 0xffffffffu ? 1u : 0u));
                } else {
                    wait_change(bar, &bar->gen, g);
                }
                st_rlx(gg, ggv + 1);
            } else {
                wait_change(bar, gg, ggv);
            }
        }
        *lds_flag = err;
    }
    __syncthreads();
}

struct DecLayer {
    const void *qkv, *wo, *gate, *up, *down;
    uint32_t t_qkv, t_wo, t_gu, t_down;
    const float *attn_norm, *ffn_norm, *bias, *q_norm, *k_norm;
    KvLayer kv;
};

struct DecParams {
    int E, F, H, HKV, HD, QR, V, n_layer, n_ctx, n_rot, neox, n_split;
    float eps, scale;
    const DecLayer *layers;
    uint32_t t_embd, t_head;
    const void *embd, *head;
    const float *out_norm, *rope;
    // The token's arena: every phase writes buffers of its own (x: 2 L + 1
    // versions of the residual), strides in floats, 256-byte aligned.
    float *x, *qkv, *att, *ffn, *part;
    int64_t sx, sqkv, satt, sffn, spart;
    float *logits;
    int *counters;  // [HKV] attention merges
    int32_t *seq, *state;
    int head_mode;  // 0: none, 1: logits, 2: logits + greedy argmax into seq[p + 1]
    GridBar *bar;
    float *best_v;
    int *best_i;
    uint64_t *trace;  // optional: workgroup 0's s_memrealtime (100 MHz) at each phase start
};

// One matvec phase for any weight type, the barrier as its pre-activation hook.
template <int MODE, class Hook>
__device__ inline void mv_phase(const MvArgs &a, int wg, int nwg, uint8_t *lds, float *red, Hook hook, float &bv,
                                int &bi) {
    // One row per wave: the kernel's register budget (two workgroups per CU)
    // holds the weights of one step and the next.
    constexpr int R = 1;
    switch (a.t) {
    case T_Q4_K: mv_run<Q4K, R, 4, MODE>(a, wg, nwg, lds, red, hook, bv, bi); break;
    case T_Q6_K: mv_run<Q6K, R, 4, MODE>(a, wg, nwg, lds, red, hook, bv, bi); break;
    default: mv_run<Q80, R, 4, MODE>(a, wg, nwg, lds, red, hook, bv, bi); break;
    }
}

__device__ inline MvArgs mv_of(uint32_t t, const void *w, const void *w2, int64_t rows, int n_in, const float *x,
                               const float *norm_w, float eps, float *y, const float *y_in = nullptr) {
    MvArgs a{};
    a.t = t, a.w = w, a.w2 = w2, a.nrows = rows, a.nb = n_in / block_values(t), a.n_in = n_in;
    a.x = x, a.norm_w = norm_w, a.eps = eps, a.y = y, a.y_in = y_in;
    return a;
}

template <int HD, int G>
__global__ __launch_bounds__(256) void k_decode(DecParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[8];
    __shared__ int flag;
    __shared__ AttnLds<HD, G> S;
    const int wg = blockIdx.x, nwg = gridDim.x;
    const int pos = p.state[0];
    float bv;
    int bi;
    int tk = 0;
    auto stamp = [&]() {
        if (p.trace && wg == 0 && threadIdx.x == 0) p.trace[tk++] = __builtin_amdgcn_s_memrealtime();
    };
    auto barrier = [&]() {
        grid_barrier(p.bar, nwg, &flag);
        stamp();
    };
    stamp();

    // Embedding (engine/src/cpu_backend.cpp:124-134), a slice per workgroup.
    {
        const int bvals = block_values(p.t_embd);
        const int nb = (p.t_embd == T_F32 || p.t_embd == T_F16) ? p.E : p.E / bvals;
        int64_t row = p.seq[pos];
        if (row < 0 || row >= p.V) row = 0;
        const int chunk = (p.E + nwg - 1) / nwg;
        const int i0 = wg * chunk, i1 = min(p.E, i0 + chunk);
        for (int i = i0 + threadIdx.x; i < i1; i += 256)
            st_dev(p.x + i, unpack_value(p.t_embd, (const uint8_t *)p.embd, (int64_t)nb * p.V, row, nb, i));
    }

    AttnArgs at{};
    at.q_stride = p.QR, at.rope = 1, at.append = 1, at.eps = p.eps, at.rope_cs = (const float2 *)p.rope;
    at.n_rot = p.n_rot, at.neox = p.neox, at.kv_per_batch = 0, at.n_ctx = p.n_ctx, at.H = p.H, at.HKV = p.HKV;
    at.n_keys = p.state, at.scale = p.scale, at.counters = p.counters;

    for (int l = 0; l < p.n_layer; l++) {
        const DecLayer &L = p.layers[l];
        float *x0 = p.x + 2 * l * p.sx, *x1 = x0 + p.sx, *x2 = x1 + p.sx;
        float *qkv = p.qkv + l * p.sqkv, *att = p.att + l * p.satt, *ffn = p.ffn + l * p.sffn;
        mv_phase<MV_STORE>(mv_of(L.t_qkv, L.qkv, nullptr, p.QR, p.E, x0, L.attn_norm, p.eps, qkv), wg, nwg, lds, red,
                           barrier, bv, bi);
        barrier();
        at.kv = L.kv, at.bias = L.bias, at.q_norm = L.q_norm, at.k_norm = L.k_norm;
        at.q = qkv, at.out = att, at.part = p.part + l * p.spart;
        for (int item = wg; item < p.HKV * p.n_split; item += nwg)
            attn_item<HD, G, 256>(at, item / p.HKV, item % p.HKV, 0, p.n_split, S);
        mv_phase<MV_ADD>(mv_of(L.t_wo, L.wo, nullptr, p.E, p.H * HD, att, nullptr, 0.f, x1, x0), wg, nwg, lds, red,
                         barrier, bv, bi);
        mv_phase<MV_GLU>(mv_of(L.t_gu, L.gate, L.up, p.F, p.E, x1, L.ffn_norm, p.eps, ffn), wg, nwg, lds, red,
                         barrier, bv, bi);
        mv_phase<MV_ADD>(mv_of(L.t_down, L.down, nullptr, p.E, p.F, ffn, nullptr, 0.f, x2, x1), wg, nwg, lds, red,
                         barrier, bv, bi);
    }
    if (p.head_mode == 0) {
        barrier();  // every workgroup has read the position
        if (wg == 0 && threadIdx.x == 0) p.state[0] = pos + 1;
        return;
    }
    const MvArgs ha = mv_of(p.t_head, p.head, nullptr, p.V, p.E, p.x + 2 * p.n_layer * p.sx, p.out_norm, p.eps,
                            p.logits);
    if (p.head_mode == 1) {
        mv_phase<MV_STORE>(ha, wg, nwg, lds, red, barrier, bv, bi);
        barrier();
        if (wg == 0 && threadIdx.x == 0) p.state[0] = pos + 1;
        return;
    }
    mv_phase<MV_ARGMAX>(ha, wg, nwg, lds, red, barrier, bv, bi);
    if (threadIdx.x == 0) {
        st_dev(p.best_v + wg, bv);
        st_dev(p.best_i + wg, bi);
    }
    barrier();
    if (wg != 0) return;
    // The first maximum over every workgroup's best (std::max_element).
    bv = -INFINITY, bi = INT_MAX;
    for (int k = threadIdx.x; k < nwg; k += 256) {
        const float v = p.best_v[k];
        const int i = p.best_i[k];
        if (v > bv || (v == bv && i < bi)) bv = v, bi = i;
    }
    best_pick_wave(bv, bi);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = bv, red[4 + (threadIdx.x >> 6)] = __int_as_float(bi);
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < 4; k++) {
            const float v = red[k];
            const int i = __float_as_int(red[4 + k]);
            if (v > bv || (v == bv && i < bi)) bv = v, bi = i;
        }
        if (bi == INT_MAX) bi = 0;  // every logit NaN
        p.state[1] = bi;
        p.seq[pos + 1] = bi;
        p.state[0] = pos + 1;
        stamp();
    }
}

// ---------------------------------------------------------------------------
template <int HD, int G>
static const void *decode_fn() {
    return (const void *)&k_decode<HD, G>;
}

static const void *decode_kernel(int HD, int G) {
#define TS5_DEC(H, GG) \
    if (HD == H && G == GG) return decode_fn<H, GG>();
    TS5_DEC(128, 1) TS5_DEC(128, 2) TS5_DEC(128, 4) TS5_DEC(128, 5) TS5_DEC(128, 7) TS5_DEC(128, 8)
    TS5_DEC(64, 1) TS5_DEC(64, 2) TS5_DEC(64, 4) TS5_DEC(64, 5) TS5_DEC(64, 7) TS5_DEC(64, 8)
#undef TS5_DEC
    return nullptr;
}

size_t decode_layer_bytes() { return sizeof(DecLayer); }
size_t decode_bar_bytes() { return sizeof(GridBar); }

// Workgroups of the persistent grid: 2 per CU when they fit (else what fits).
int decode_grid(int HD, int G, int n_cu, size_t lds_bytes) {
    const void *f = decode_kernel(HD, G);
    if (!f) return 0;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, 256, lds_bytes) != hipSuccess) return 0;
    return (per_cu >= 2 ? 2 : per_cu) * n_cu;
}

hipError_t fill_decode_layer(void *dst, const DecodeLayerIn &in) {
    DecLayer L{};
    L.qkv = in.qkv, L.wo = in.wo, L.gate = in.gate, L.up = in.up, L.down = in.down;
    L.t_qkv = in.t_qkv, L.t_wo = in.t_wo, L.t_gu = in.t_gu, L.t_down = in.t_down;
    L.attn_norm = in.attn_norm, L.ffn_norm = in.ffn_norm, L.bias = in.bias, L.q_norm = in.q_norm;
    L.k_norm = in.k_norm, L.kv = in.kv;
    std::memcpy(dst, &L, sizeof L);
    return hipSuccess;
}

hipError_t launch_decode(const DecodeIn &in, hipStream_t s) {
    const void *f = decode_kernel(in.HD, in.H / in.HKV);
    if (!f) return hipErrorInvalidValue;
    DecParams p{};
    p.E = in.E, p.F = in.F, p.H = in.H, p.HKV = in.HKV, p.HD = in.HD, p.QR = (in.H + 2 * in.HKV) * in.HD;
    p.V = in.V, p.n_layer = in.n_layer, p.n_ctx = in.n_ctx, p.n_rot = in.n_rot, p.neox = in.neox;
    p.n_split = in.n_split, p.eps = in.eps, p.scale = in.scale, p.layers = (const DecLayer *)in.layers;
    p.t_embd = in.t_embd, p.t_head = in.t_head, p.embd = in.embd, p.head = in.head, p.out_norm = in.out_norm;
    p.rope = in.rope, p.x = in.x, p.qkv = in.qkv, p.att = in.att, p.ffn = in.ffn, p.logits = in.logits;
    p.part = in.part, p.sx = in.sx, p.sqkv = in.sqkv, p.satt = in.satt, p.sffn = in.sffn, p.spart = in.spart;
    p.counters = in.counters, p.seq = in.seq, p.state = in.state, p.head_mode = in.head_mode;
    p.bar = (GridBar *)in.bar, p.best_v = in.best_v, p.best_i = in.best_i, p.trace = in.trace;
    void *args[] = {&p};
    return hipLaunchCooperativeKernel(f, dim3(in.grid), dim3(256), args, in.lds_bytes, s);
}

}  // namespace ts5hip
