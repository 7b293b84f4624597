// One decode token as one persistent kernel with a weight stream.
//
// Every workgroup (one per CU, 512 threads) stays resident for the whole
// token. The token is a program of phases, built on the host:
//   embed            x0 = row seq[p] of token_embd (each workgroup a slice)
//   per layer        QKV matvec (rmsnorm fused) | attention (RoPE, q8 append,
//                    split-K, merge) | O matvec (x +=) | gate/up + SiLU
//                    (rmsnorm fused) | down matvec (x +=)
//   head             logits = W_out rmsnorm(x) [+ greedy argmax -> seq[p+1]]
// and then state[0] = p + 1.
//
// Weight stream. A matvec phase's rows are cut into slots of whole rows (at
// most SLOT_BYTES of weights each); workgroup w owns a contiguous run of each
// phase's slots. Its slots, phase after phase, form one stream that runs
// through a ring of RING_SLOTS slots in LDS: global_load_lds_dwordx4 moves
// 16 bytes per lane straight from HBM into the ring (no registers), each
// wave issuing the same SLOT_LOADS instructions per slot, so `s_waitcnt
// vmcnt(SLOT_LOADS * k)` tells a wave that its part of a slot has landed
// while the k slots issued after it are still in flight (vector memory loads
// return in order). The stream does not stop at phase changes: while a
// workgroup waits for a phase's input, that phase's first slots are already
// on their way.
//
// Phase hand-off without grid barriers. Every value that crosses workgroups
// (x, q|k|v, attention partials and output, the FFN activation, each
// workgroup's final word) is a 64-bit word (value bits, launch tag) written
// with one device-coherent store. A reader takes a word with an ordinary load
// and accepts it when its tag is this launch's tag; otherwise it polls the
// word with device-coherent loads, which do not hit a stale cached copy.
// Nothing waits for stores to complete, so nothing drains the weight stream.
// Every phase writes buffers of its own (the arena): a word is written once
// per launch, and the tag (launches so far + 1) tells this launch's words
// from the previous ones.
//
// Termination: the grid is launched cooperatively (every workgroup resident).
// A poll that outlasts a bounded spin count sets the error flag; polls that
// see the flag give up at once, so the kernel always exits and the host
// reports the error.
#include <algorithm>
#include <cstring>

#include "attn_core.h"
#include "kernels.h"
#include "mv_core.h"

namespace ts5hip {

constexpr int DEC_NT = 512, DEC_WAVES = DEC_NT / WAVE;
constexpr int RING_SLOTS = 3, SLOT_BYTES = 32768;
constexpr int SLOT_LOADS = SLOT_BYTES / (16 * DEC_NT);  // DMA instructions per wave per slot
constexpr int YIN_MAX = 1024;                            // rows of one matrix phase per workgroup
static_assert(SLOT_LOADS * 16 * DEC_NT == SLOT_BYTES, "a slot is whole DMA rounds");

// One phase of the token program (device copy made by fill_decode_phase).
struct DPhase {
    int kind, t, ne0, nb, nrows, rps, nslots, body_row;  // body_row: bytes of one row's block bodies
    const uint8_t *w, *w2;  // block bodies (w2: the up projection of GLU)
    const uint8_t *s, *s2;  // f16 block scales of split layouts (Q6_K, Q8_0), else null
    const uint64_t *x;      // tagged input
    const float *norm_w;
    uint64_t *y;            // tagged output
    const uint64_t *y_in;   // ADD: tagged residual
    float *logits;          // LOGITS
    KvLayer kv;             // ATTN
    const float *bias, *q_norm, *k_norm;
    uint64_t *part;  // ATTN: tagged partials [n_split][H][HD + 2]
};

// The kernel reads the program through the constant address space: the
// records are never written while it runs, so uniform reads become scalar
// loads (a vector load would make the wave wait for every weight DMA in
// flight before it, since vector memory loads complete in order).
typedef const __attribute__((address_space(4))) DPhase CPhase;

// Device words of the persistent kernel, zeroed with the arena.
struct DecSync {
    int err;       // a poll gave up
    int launches;  // tokens run so far (the next launch's tag is launches + 1)
    int pad[62];
};

struct DecParams {
    CPhase *ph;
    int n_ph;
    int E, H, HKV, V, n_ctx, n_rot, neox, n_split;
    float eps, scale;
    uint32_t t_embd;
    const void *embd;
    const float2 *rope;
    uint64_t *x0;
    int32_t *seq, *state;  // state[0] position, [1] greedy id
    int head_mode;         // 0: none, 1: logits, 2: logits + greedy argmax into seq[p + 1]
    uint64_t *best;        // [2][grid] tagged (value, row) of each workgroup; also its done-word
    DecSync *sync;
    uint64_t *trace;       // optional: workgroup 0's s_memrealtime at each phase start
    int act_off, yin_off;  // LDS layout (bytes)
};

// ---------------------------------------------------------------------------
// Tagged words.
// ---------------------------------------------------------------------------
constexpr unsigned SPIN_LIMIT = 1u << 21;

__device__ inline void st_tag(uint64_t *p, uint32_t bits, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void st_tagf(uint64_t *p, float v, uint32_t tag) { st_tag(p, __float_as_uint(v), tag); }
__device__ inline bool tag_ok(uint64_t w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }

// Polls *p (last read as w) until its tag matches; gives up when the error
// flag is set, or sets it after the spin limit.
__device__ __noinline__ uint64_t poll_tag(const uint64_t *p, uint64_t w, uint32_t tag, int *err) {
    unsigned spins = 0;
    while (!tag_ok(w, tag)) {
        __builtin_amdgcn_s_sleep(2);
        w = __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((++spins & 63) == 0) {
            if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) break;
            if (spins > SPIN_LIMIT) {
                __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    return w;
}
__device__ inline uint32_t ld_tag(const uint64_t *p, uint32_t tag, int *err) {
    uint64_t w = *p;
    if (!tag_ok(w, tag)) w = poll_tag(p, w, tag, err);
    return (uint32_t)w;
}
__device__ inline float ld_tagf(const uint64_t *p, uint32_t tag, int *err) {
    return __uint_as_float(ld_tag(p, tag, err));
}

// ---------------------------------------------------------------------------
// The weight ring.
// ---------------------------------------------------------------------------
// dma16 (mv_core.h): 64 lanes x 16 bytes from per-lane global addresses to
// LDS [base, base+1024), by inline asm so that the compiler does not wait for
// these loads (it would wait for every LDS DMA before any LDS read); the
// stream's waits are explicit.
// Workgroup barrier that also completes this wave's LDS reads before it.
__device__ inline void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// Stores through inline asm, so that each is exactly one instruction in the
// count below.
__device__ inline void st_tag_asm(uint64_t *p, float v, uint32_t tag) {
    const uint64_t w = ((uint64_t)tag << 32) | __float_as_uint(v);
    asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(p), "v"(w) : "memory");
}
__device__ inline void st_f32_asm(float *p, float v) { asm volatile("global_store_dword %0, %1, off" ::"v"(p), "v"(v) : "memory"); }

// s_waitcnt vmcnt(n) for a wave-uniform n (at most 15; fewer is only slower).
__device__ inline void wait_vm(int n) {
    switch (__builtin_amdgcn_readfirstlane(n)) {
#define TS5_W(N) \
    case N: asm volatile("s_waitcnt vmcnt(" #N ")" ::: "memory"); break;
        TS5_W(0) TS5_W(1) TS5_W(2) TS5_W(3) TS5_W(4) TS5_W(5) TS5_W(6) TS5_W(7) TS5_W(8) TS5_W(9) TS5_W(10)
        TS5_W(11) TS5_W(12) TS5_W(13) TS5_W(14)
#undef TS5_W
    default: asm volatile("s_waitcnt vmcnt(15)" ::: "memory"); break;
    }
}

struct SlotGeom {
    int r0, nr;
    int64_t boff;  // byte offset of row r0's bodies
    int nbody;     // 16-byte pieces of one matrix's bodies
    int delta;     // split scales: byte of row r0's first scale within its 16-byte piece
    int nsc;       // ... and the pieces they span
    int64_t soff;  // 16-byte aligned byte offset of that piece
};
__device__ inline SlotGeom slot_geom(CPhase &P, int j) {
    SlotGeom g;
    g.r0 = j * P.rps;
    g.nr = min(P.rps, P.nrows - g.r0);
    g.boff = (int64_t)g.r0 * P.body_row;
    g.nbody = g.nr * P.body_row / 16;
    g.delta = 0, g.nsc = 0, g.soff = 0;
    if (P.s) {
        const int64_t b0 = 2 * (int64_t)g.r0 * P.nb;
        g.soff = b0 & ~(int64_t)15;
        g.delta = (int)(b0 - g.soff);
        g.nsc = (g.delta + 2 * g.nr * P.nb + 15) / 16;
    }
    return g;
}

// Issues slot j of phase P into the ring slot at LDS byte address dst. A
// slot holds, in 16-byte pieces: the bodies of w, of w2 (GLU), the scales of
// w, of w2 (split layouts). Lanes past the end re-read the first piece into
// the slot's unused tail, so every wave issues exactly SLOT_LOADS loads.
__device__ inline void issue_slot(CPhase &P, int j, uint32_t dst) {
    const SlotGeom g = slot_geom(P, j);
    const bool glu = P.kind == DPH_GLU;
    const int c0 = g.nbody, c1 = c0 + (glu ? g.nbody : 0), c2 = c1 + g.nsc, c3 = c2 + (glu ? g.nsc : 0);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < SLOT_LOADS; k++) {
        const int rnd = k * DEC_WAVES + wave, q = rnd * 64 + lane;
        const uint8_t *src = P.w + g.boff;
        if (q < c0) src = P.w + g.boff + 16 * (int64_t)q;
        else if (q < c1) src = P.w2 + g.boff + 16 * (int64_t)(q - c0);
        else if (q < c2) src = P.s + g.soff + 16 * (int64_t)(q - c1);
        else if (q < c3) src = P.s2 + g.soff + 16 * (int64_t)(q - c2);
        dma16(src, __builtin_amdgcn_readfirstlane(dst + rnd * 1024));
    }
}

// This workgroup's slots [lo, hi) of a phase.
__device__ inline void my_slots(CPhase &P, int wg, int nwg, int &lo, int &hi) {
    lo = (int)((int64_t)P.nslots * wg / nwg);
    hi = (int)((int64_t)P.nslots * (wg + 1) / nwg);
}

// Wave-uniform values the compiler cannot prove uniform (they live across
// loops with per-lane exits) go through readfirstlane: uniform indices keep
// the phase records on scalar loads.
__device__ inline int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Stream cursor: the next (phase, slot) this workgroup issues.
struct Cursor {
    int ph, j, hi;
};
__device__ inline void cursor_seek(const DecParams &p, Cursor &c, int ph, int wg, int nwg) {
    for (ph = uni(ph); ph < p.n_ph; ph++) {
        CPhase &P = p.ph[ph];
        if (P.kind == DPH_ATTN) continue;
        int lo, hi;
        my_slots(P, wg, nwg, lo, hi);
        if (lo < hi) {
            c.ph = uni(ph), c.j = uni(lo), c.hi = uni(hi);
            return;
        }
    }
    c.ph = p.n_ph, c.j = 0, c.hi = 0;
}

// ---------------------------------------------------------------------------
// Activation prologue over a tagged input: the quantized activation of
// build_act (mv_core.h), one 16-value run per thread and round, two rounds.
// ---------------------------------------------------------------------------
__device__ inline void build_act_tagged(const uint64_t *x, const float *norm_w, float eps, int n, const Act &a,
                                        float *red, uint32_t tag, int *err) {
    constexpr int NT = DEC_NT, RMAX = 2;  // n <= 16 * NT * RMAX
    float v[RMAX][16];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < RMAX; k++) {
        const int r = threadIdx.x + NT * k;
        if (r < n / 16) {
            uint64_t w[16];
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint4 u = *(const uint4 *)(x + 16 * r + 2 * e);
                w[2 * e] = ((uint64_t)u.y << 32) | u.x;
                w[2 * e + 1] = ((uint64_t)u.w << 32) | u.z;
            }
#pragma unroll
            for (int e = 0; e < 16; e++) {
                if (!tag_ok(w[e], tag)) w[e] = poll_tag(x + 16 * r + e, w[e], tag, err);
                v[k][e] = __uint_as_float((uint32_t)w[e]);
                ss += v[k][e] * v[k][e];
            }
        }
    }
    float s = 1.0f;
    if (norm_w) {
        ss = wave_sum(ss);
        if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
        __syncthreads();
        ss = 0.f;
#pragma unroll
        for (int w = 0; w < NT / 64; w++) ss += red[w];
        s = 1.0f / sqrtf(ss / (float)n + eps);
    }
#pragma unroll
    for (int k = 0; k < RMAX; k++) {
        const int r = threadIdx.x + NT * k;
        if (r >= n / 16) continue;
        if (norm_w) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 wv = *(const float4 *)(norm_w + 16 * r + 4 * q);
                v[k][4 * q] = v[k][4 * q] * s * wv.x;
                v[k][4 * q + 1] = v[k][4 * q + 1] * s * wv.y;
                v[k][4 * q + 2] = v[k][4 * q + 2] * s * wv.z;
                v[k][4 * q + 3] = v[k][4 * q + 3] * s * wv.w;
            }
        }
        float amax = 0.f, sum = 0.f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            amax = fmaxf(amax, fabsf(v[k][i]));
            sum += v[k][i];
        }
        amax = fmaxf(amax, __shfl_xor(amax, 1, WAVE));  // runs 2g and 2g+1 are adjacent lanes
        sum += __shfl_xor(sum, 1, WAVE);
        const float inv = amax > 0.f ? 16383.0f / amax : 0.f;
        uint32_t hw[4], lw[4];
        int is = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            uint32_t h = 0, l = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int x16 = max(-16383, min(16383, (int)rintf(v[k][4 * q + e] * inv)));
                const int lo = (int)(int8_t)(x16 & 255);
                const int hi = (x16 - lo) >> 8;
                h |= (uint32_t)(hi & 255) << (8 * e);
                l |= (uint32_t)(lo & 255) << (8 * e);
                is += x16;
            }
            hw[q] = h, lw[q] = l;
        }
        *(uint4 *)(a.hi + 16 * r) = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        *(uint4 *)(a.lo + 16 * r) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        a.isum[r] = is;
        if ((r & 1) == 0) {
            a.scale[r / 2] = amax / 16383.0f;
            a.sum[r / 2] = sum;
        }
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// The stream's state. Loads return in order, so a slot has landed once no
// more vector memory instructions are outstanding than this wave issued after
// it: SLOT_LOADS per later slot, plus the `kst` output stores of the last
// phase end when the slot went out before them (`nbefore` counts those
// slots). Instructions this count misses (the compiler's own loads and
// stores outside the slot loop) only make a wait longer.
// ---------------------------------------------------------------------------
struct Stream {
    Cursor ic;
    int issued = 0, consumed = 0, nbefore = 0, kst = 0;
};

__device__ __attribute__((always_inline)) inline void stream_issue(const DecParams &p, Stream &st, uint32_t ring,
                                                                   int wg, int nwg) {
    st.ic.ph = uni(st.ic.ph), st.ic.j = uni(st.ic.j), st.ic.hi = uni(st.ic.hi);
    if (st.ic.ph >= p.n_ph) return;
    issue_slot(p.ph[st.ic.ph], st.ic.j, ring + (uni(st.issued) % RING_SLOTS) * SLOT_BYTES);
    st.issued = uni(st.issued + 1);
    if (++st.ic.j == st.ic.hi) cursor_seek(p, st.ic, st.ic.ph + 1, wg, nwg);
}

// Waits for the oldest slot in flight and hands it out.
__device__ __attribute__((always_inline)) inline int stream_take(Stream &st) {
    st.consumed = uni(st.consumed), st.issued = uni(st.issued), st.nbefore = uni(st.nbefore);
    wait_vm(SLOT_LOADS * (st.issued - st.consumed - 1) + (st.nbefore > 0 ? st.kst : 0));
    if (st.nbefore > 0) st.nbefore--;
    return st.consumed++ % RING_SLOTS;
}

// ---------------------------------------------------------------------------
// A matrix phase: this workgroup's slots [lo, hi), each waited for, then the
// next slot of the stream issued, then computed from the ring into `out`
// (LDS, one value per row of the workgroup's range, stored at the phase end).
//
// Lanes split a row's blocks as in the standalone matvec (mv_core.h); a row
// of nb blocks takes npass = nb / (64 / LPB) sweeps (rounded up to 1, 2, 4 or
// 8). Wave w always takes sweep w % npass, so it builds its activation
// fragment in registers once per phase; rows go to the 8 / npass waves of
// each sweep in turn, and with npass > 1 the sweeps' partial sums meet in LDS.
// ---------------------------------------------------------------------------
constexpr int PART_ROWS = 32;  // rows per slot of a phase with npass > 1

template <int KIND>
__device__ inline void put_row(float *out, int r, float acc, float acc2, bool store, float &bv, int &bi, int row) {
    if (KIND == DPH_ARGMAX && (acc > bv || (acc == bv && row < bi))) bv = acc, bi = row;
    if (!store) return;
    out[r] = KIND == DPH_GLU ? acc / (1.0f + expf(-acc)) * acc2 : acc;  // cpu_backend.cpp:260-261
}

template <class F, int KIND>
__device__ inline void run_phase(const DecParams &p, CPhase &P, int lo, int hi, const CAct &x, float *out, int row0,
                                 float &bv, int &bi, const uint8_t *lds, Stream &st, uint32_t ring, int wg, int nwg,
                                 float *part_s, uint64_t &waited) {
    constexpr int BPI = WAVE / F::LPB;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, bsub = lane / F::LPB, sub = lane % F::LPB;
    const int nb = P.nb, br = P.body_row;
    const int sweeps = (nb + BPI - 1) / BPI;
    const int npass = sweeps <= 1 ? 1 : sweeps <= 2 ? 2 : sweeps <= 4 ? 4 : 8;
    const int k = wave % npass, rw = wave / npass, rpr = DEC_WAVES / npass;
    const int b = bsub + BPI * k;
    const bool bin = b < nb;
    typename F::X xf;
    if (bin) xf = F::load_x(x, b, sub);
    for (int j = uni(lo); j < hi; j = uni(j + 1)) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        const int rs = stream_take(st);
        lds_barrier();
        waited += __builtin_amdgcn_s_memrealtime() - t0;
        const uint8_t *slot = lds + rs * SLOT_BYTES;
        stream_issue(p, st, ring, wg, nwg);
        const SlotGeom g = slot_geom(P, j);
        const uint8_t *w2b = slot + g.nr * br;
        const uint8_t *sc1 = slot + (KIND == DPH_GLU ? 2 : 1) * g.nr * br + g.delta;
        const uint8_t *sc2 = sc1 + 16 * g.nsc;
        for (int i = rw; i < g.nr; i += rpr) {
            float acc = 0.f, acc2 = 0.f;
            if (bin) {
                acc = F::dot(F::load_w_lds(slot + i * br, sc1 + 2 * i * nb, b, sub), xf, sub);
                if (KIND == DPH_GLU) acc2 = F::dot(F::load_w_lds(w2b + i * br, sc2 + 2 * i * nb, b, sub), xf, sub);
            }
            acc = wave_sum_dpp(acc);
            if (KIND == DPH_GLU) acc2 = wave_sum_dpp(acc2);
            if (npass == 1) {
                put_row<KIND>(out, g.r0 + i - row0, acc, acc2, lane == 0, bv, bi, g.r0 + i);
            } else if (lane == 0) {
                part_s[(i * DEC_WAVES + k) * 2] = acc;
                part_s[(i * DEC_WAVES + k) * 2 + 1] = acc2;
            }
        }
        if (npass > 1) {
            lds_barrier();
            if (threadIdx.x < g.nr) {
                const int i = threadIdx.x;
                float a = 0.f, a2 = 0.f;
                for (int q = 0; q < npass; q++) a += part_s[(i * DEC_WAVES + q) * 2], a2 += part_s[(i * DEC_WAVES + q) * 2 + 1];
                put_row<KIND>(out, g.r0 + i - row0, a, a2, true, bv, bi, g.r0 + i);
            }
        }
    }
}

template <class F>
__device__ inline void run_phase_kind(int kind, const DecParams &p, CPhase &P, int lo, int hi, const CAct &x,
                                      float *out, int row0, float &bv, int &bi, const uint8_t *lds, Stream &st,
                                      uint32_t ring, int wg, int nwg, float *part_s, uint64_t &waited) {
    switch (kind) {
    case DPH_MV: run_phase<F, DPH_MV>(p, P, lo, hi, x, out, row0, bv, bi, lds, st, ring, wg, nwg, part_s, waited); break;
    case DPH_ADD: run_phase<F, DPH_ADD>(p, P, lo, hi, x, out, row0, bv, bi, lds, st, ring, wg, nwg, part_s, waited); break;
    case DPH_GLU: run_phase<F, DPH_GLU>(p, P, lo, hi, x, out, row0, bv, bi, lds, st, ring, wg, nwg, part_s, waited); break;
    case DPH_LOGITS: run_phase<F, DPH_LOGITS>(p, P, lo, hi, x, out, row0, bv, bi, lds, st, ring, wg, nwg, part_s, waited); break;
    default: run_phase<F, DPH_ARGMAX>(p, P, lo, hi, x, out, row0, bv, bi, lds, st, ring, wg, nwg, part_s, waited); break;
    }
}

// ---------------------------------------------------------------------------
// Attention over tagged words: the work items of the standalone kernel
// (attn_core.h); the partials go out tagged, and the workgroup that ran
// split 0 of a KV head merges it once every split's record has arrived
// (attn_merge.comp:18-47).
// ---------------------------------------------------------------------------
template <int HD, int G>
__device__ inline void attn_items(const DecParams &p, CPhase &P, AttnLds<HD, G> &S, int wg, int nwg,
                                  uint32_t tag) {
    constexpr int NT = DEC_NT, NPAIR = G * HD / 2, PPT = AttnShape<HD, G, NT>::PPT;
    const int tid = threadIdx.x;
    int *err = &p.sync->err;
    AttnArgs at{};
    at.q_stride = 0, at.rope = 1, at.append = 1, at.eps = p.eps, at.rope_cs = p.rope;
    at.n_rot = p.n_rot, at.neox = p.neox, at.kv_per_batch = 0, at.n_ctx = p.n_ctx, at.H = p.H, at.HKV = p.HKV;
    at.n_keys = p.state, at.scale = p.scale, at.kv = KvLayer{P.kv.k, P.kv.ks, P.kv.v, P.kv.vs};
    at.bias = P.bias, at.q_norm = P.q_norm;
    at.k_norm = P.k_norm;
    const int64_t rec = HD + 2, sstride = (int64_t)p.H * rec;
    const int n_split = p.n_split;
    for (int item = wg; item < p.HKV * n_split; item += nwg) {
        const int split = item / p.HKV, kvh = item % p.HKV;
        const AttnSpan sp = attn_span(at, split, kvh, 0, n_split);
        attn_prepare<HD, G, NT>(at, kvh, sp, S, [&](int64_t e) { return ld_tagf(P.x + e, tag, err); });
        float o[PPT][2];
        attn_tiles<HD, G, NT>(at, sp, S, o);
        uint64_t *pb = P.part + split * sstride + (int64_t)kvh * G * rec;
#pragma unroll
        for (int k = 0; k < PPT; k++) {
            const int pp = tid + NT * k;
            if (pp < NPAIR) {
                const int gg = (2 * pp) / HD, d = (2 * pp) % HD;
                st_tagf(pb + gg * rec + d, o[k][0], tag);
                st_tagf(pb + gg * rec + d + 1, o[k][1], tag);
            }
        }
        if (tid < G) {
            st_tagf(pb + tid * rec + HD, S.m_s[tid], tag);
            st_tagf(pb + tid * rec + HD + 1, S.l_s[tid], tag);
        }
        __syncthreads();  // S is reused by the next item
    }
}

// Workgroup kvh ran item kvh = (split 0, kvh), and its other items, first.
template <int HD, int G>
__device__ inline void attn_merges(const DecParams &p, CPhase &P, AttnLds<HD, G> &S, int wg, int nwg, uint32_t tag) {
    constexpr int NT = DEC_NT;
    const int tid = threadIdx.x;
    int *err = &p.sync->err;
    const int64_t rec = HD + 2, sstride = (int64_t)p.H * rec;
    const int n_split = p.n_split;
    for (int kvh = wg; kvh < p.HKV; kvh += nwg) {
        const uint64_t *pa = P.part + (int64_t)kvh * G * rec;
        for (int j = tid; j < n_split * G; j += NT) {
            const int sp = j / G, gg = j % G;
            S.mw[sp][gg] = ld_tagf(pa + sp * sstride + gg * rec + HD, tag, err);
            S.lw[sp][gg] = ld_tagf(pa + sp * sstride + gg * rec + HD + 1, tag, err);
        }
        __syncthreads();
        if (tid < G) {
            float M = -INFINITY;
            for (int sp = 0; sp < n_split; sp++) M = fmaxf(M, S.mw[sp][tid]);
            float L = 0.f;
            for (int sp = 0; sp < n_split; sp++) {
                const float m = S.mw[sp][tid];
                const float w = m == -INFINITY ? 0.f : expf(m - M);
                S.mw[sp][tid] = w;
                L += w * S.lw[sp][tid];
            }
            S.red[tid] = L;
        }
        __syncthreads();
        for (int j = tid; j < G * HD; j += NT) {
            const int gg = j / HD, d = j % HD;
            const uint64_t *pd = pa + gg * rec + d;
            float acc = 0.f;
#pragma unroll 8
            for (int sp = 0; sp < n_split; sp++) acc += S.mw[sp][gg] * ld_tagf(pd + sp * sstride, tag, err);
            st_tagf(P.y + (int64_t)(kvh * G + gg) * HD + d, acc / S.red[gg], tag);
        }
        __syncthreads();
    }
}

// (v, i) of a workgroup: every wave's best, first maximum (lower row on ties).
__device__ inline void best_pick_wg(float &v, int &i, float *red) {
    best_pick_wave(v, i);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v, red[DEC_WAVES + (threadIdx.x >> 6)] = __int_as_float(i);
    __syncthreads();
    for (int k = 0; k < DEC_WAVES; k++) {
        const float w = red[k];
        const int j = __float_as_int(red[DEC_WAVES + k]);
        if (w > v || (w == v && j < i)) v = w, i = j;
    }
}

template <int HD, int G>
__global__ __launch_bounds__(DEC_NT) void k_decode(DecParams p) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[2 * DEC_WAVES];
    __shared__ float part_s[PART_ROWS * DEC_WAVES * 2];
    const int wg = blockIdx.x, nwg = gridDim.x;
    const int pos = p.state[0];
    const uint32_t tag = (uint32_t)p.sync->launches + 1u;
    int *err = &p.sync->err;
    const uint32_t ring = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)lds;
    uint8_t *act_lds = lds + p.act_off;
    float *yin = (float *)(lds + p.yin_off);
    float *out_s = yin + YIN_MAX;
    AttnLds<HD, G> &S = *(AttnLds<HD, G> *)act_lds;  // the attention phase and the activation never overlap
    // Profile: every workgroup's s_memrealtime (100 MHz) at [k][e], k = 0 the
    // embedding, 1 + ph the phases, n_ph + 1 the end; e = start, input ready,
    // done, and [k][3] the ticks spent waiting for weight slots.
    auto stamp = [&](int k, int e) {
        if (p.trace && threadIdx.x == 0)
            p.trace[((size_t)wg * (p.n_ph + 2) + k) * 4 + e] = __builtin_amdgcn_s_memrealtime();
    };
    stamp(0, 0);

    // The stream: the first RING_SLOTS - 1 slots go out before anything else.
    Stream st;
    cursor_seek(p, st.ic, 0, wg, nwg);
    for (int k = 0; k < RING_SLOTS - 1; k++) stream_issue(p, st, ring, wg, nwg);

    // Embedding (engine/src/cpu_backend.cpp:124-134), a slice per workgroup.
    {
        const int nb = (p.t_embd == T_F32 || p.t_embd == T_F16) ? p.E : p.E / block_values(p.t_embd);
        int64_t row = p.seq[pos];
        if (row < 0 || row >= p.V) row = 0;
        const int chunk = (p.E + nwg - 1) / nwg;
        const int i0 = wg * chunk, i1 = min(p.E, i0 + chunk);
        for (int i = i0 + threadIdx.x; i < i1; i += DEC_NT)
            st_tagf(p.x0 + i, unpack_value(p.t_embd, (const uint8_t *)p.embd, (int64_t)nb * p.V, row, nb, i), tag);
    }
    stamp(0, 2);

    float bv = -INFINITY;
    int bi = INT_MAX;
    for (int ph = 0; ph < p.n_ph; ph++) {
        CPhase &P = p.ph[ph];
        stamp(1 + ph, 0);
        if (P.kind == DPH_ATTN) {
            attn_items<HD, G>(p, P, S, wg, nwg, tag);
            stamp(1 + ph, 1);
            attn_merges<HD, G>(p, P, S, wg, nwg, tag);
            stamp(1 + ph, 2);
            continue;
        }
        int lo, hi;
        my_slots(P, wg, nwg, lo, hi);
        if (lo >= hi) continue;
        const int row0 = lo * P.rps, row1 = min(P.nrows, hi * P.rps);
        if (P.kind == DPH_ADD)
            for (int r = row0 + threadIdx.x; r < row1; r += DEC_NT) yin[r - row0] = ld_tagf(P.y_in + r, tag, err);
        const Act xa = act_view(act_lds, P.ne0);
        build_act_tagged(P.x, P.norm_w, p.eps, P.ne0, xa, red, tag, err);
        stamp(1 + ph, 1);
        const CAct x{xa.hi, xa.lo, xa.scale, xa.sum, xa.isum};
        const int kind = (P.kind == DPH_LOGITS && p.head_mode == 2) ? DPH_ARGMAX : P.kind;
        uint64_t waited = 0;
        switch (P.t) {
        case T_Q4_K: run_phase_kind<Q4K>(kind, p, P, lo, hi, x, out_s, row0, bv, bi, lds, st, ring, wg, nwg, part_s, waited); break;
        case T_Q6_K: run_phase_kind<Q6K>(kind, p, P, lo, hi, x, out_s, row0, bv, bi, lds, st, ring, wg, nwg, part_s, waited); break;
        default: run_phase_kind<Q80>(kind, p, P, lo, hi, x, out_s, row0, bv, bi, lds, st, ring, wg, nwg, part_s, waited); break;
        }
        // The phase's outputs, row0..row1, one coalesced round of stores; the
        // slots still in flight were issued before them.
        lds_barrier();
        int n_st = 0;
        for (int r = row0 + (int)threadIdx.x; r < row1; r += DEC_NT, n_st++) {
            const float v = out_s[r - row0];
            if (P.kind == DPH_LOGITS) st_f32_asm(P.logits + r, v);
            else st_tag_asm(P.y + r, P.kind == DPH_ADD ? yin[r - row0] + v : v, tag);
        }
        // Every lane of a wave runs the loop as often as its lane 0 (the first row).
        st.kst = uni(n_st);
        st.nbefore = uni(st.issued - st.consumed);
        stamp(1 + ph, 2);
        if (p.trace && threadIdx.x == 0) p.trace[((size_t)wg * (p.n_ph + 2) + 1 + ph) * 4 + 3] = waited;
        lds_barrier();  // the activation, residual and output rows are rebuilt by the next phase
    }

    // Each workgroup's best (value, row), which also says that it is done;
    // workgroup 0 takes the first maximum over all of them
    // (std::max_element) and ends the token.
    if (p.head_mode == 2) best_pick_wg(bv, bi, red);
    if (threadIdx.x == 0) {
        st_tag(p.best + wg, __float_as_uint(bv), tag);
        st_tag(p.best + nwg + wg, (uint32_t)bi, tag);
    }
    stamp(p.n_ph + 1, 0);
    if (wg != 0) return;
    bv = -INFINITY, bi = INT_MAX;
    for (int k = threadIdx.x; k < nwg; k += DEC_NT) {
        const float v = ld_tagf(p.best + k, tag, err);
        const int i = (int)ld_tag(p.best + nwg + k, tag, err);
        if (v > bv || (v == bv && i < bi)) bv = v, bi = i;
    }
    best_pick_wg(bv, bi, red);
    if (threadIdx.x == 0) {
        if (p.head_mode == 2) {
            if (bi == INT_MAX || bi < 0) bi = 0;  // every logit NaN
            p.state[1] = bi;
            p.seq[pos + 1] = bi;
        }
        p.sync->launches = (int)tag;
        p.state[0] = pos + 1;
    }
    stamp(p.n_ph + 1, 2);
}

// ---------------------------------------------------------------------------
template <int HD, int G>
static const void *decode_fn() {
    return (const void *)&k_decode<HD, G>;
}

#define TS5_DEC_SHAPES(X) \
    X(128, 1) X(128, 2) X(128, 4) X(128, 5) X(128, 7) X(128, 8) X(64, 1) X(64, 2) X(64, 4) X(64, 5) X(64, 7) X(64, 8)

static const void *decode_kernel(int HD, int G) {
#define TS5_DEC(H, GG) \
    if (HD == H && G == GG) return decode_fn<H, GG>();
    TS5_DEC_SHAPES(TS5_DEC)
#undef TS5_DEC
    return nullptr;
}

static size_t attn_lds_bytes(int HD, int G) {
#define TS5_DEC(H, GG) \
    if (HD == H && G == GG) return sizeof(AttnLds<H, GG>);
    TS5_DEC_SHAPES(TS5_DEC)
#undef TS5_DEC
    return 0;
}

static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }
static size_t act_region(int HD, int G, int max_in) { return al256(std::max(act_bytes(max_in), attn_lds_bytes(HD, G))); }

size_t decode_phase_bytes() { return sizeof(DPhase); }
size_t decode_sync_bytes() { return sizeof(DecSync); }

// LDS of the kernel: the ring, the activation (or attention) region, the
// residual rows and the output rows of a matrix phase. 0: no kernel for this head shape.
size_t decode_lds_bytes(int HD, int G, int max_in) {
    if (!attn_lds_bytes(HD, G)) return 0;
    return (size_t)RING_SLOTS * SLOT_BYTES + act_region(HD, G, max_in) + 8 * YIN_MAX;
}

// One workgroup per CU, all resident; 0 when the kernel does not fit.
int decode_grid(int HD, int G, int n_cu, size_t lds_bytes) {
    const void *f = decode_kernel(HD, G);
    if (!f || lds_bytes > 160 * 1024) return 0;
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, f, DEC_NT, lds_bytes) != hipSuccess) return 0;
    return per_cu >= 1 ? n_cu : 0;
}

// Rows per slot: as many whole rows as a slot holds, then as few as keep the
// same number of slots on the busiest workgroup. 0: one row does not fit.
// With npass sweeps per row, rows go in rounds of 8 / npass: a multiple of
// that when a slot holds as many.
static int rows_per_slot(int row_bytes, int nrows, int grid, int round) {
    int cap = (SLOT_BYTES - 64) / row_bytes;
    if (cap < 1) return 0;
    if (cap >= round) cap -= cap % round;
    const int64_t per = ((int64_t)(nrows + cap - 1) / cap + grid - 1) / grid;
    int rps = (int)std::max<int64_t>(1, (nrows + per * grid - 1) / (per * grid));
    if (rps > round && rps % round) rps = std::min(cap, rps + round - rps % round);
    return rps;
}

int fill_decode_phase(void *dst, const DecodePhaseIn &in, int grid) {
    DPhase P{};
    P.kind = in.kind, P.t = (int)in.t, P.ne0 = in.ne0, P.nrows = in.nrows;
    P.x = (const uint64_t *)in.x, P.norm_w = in.norm_w, P.y = (uint64_t *)in.y, P.y_in = (const uint64_t *)in.y_in;
    P.logits = in.logits, P.kv = in.kv, P.bias = in.bias, P.q_norm = in.q_norm, P.k_norm = in.k_norm;
    P.part = (uint64_t *)in.part;
    if (in.kind != DPH_ATTN) {
        if (in.t != T_Q4_K && in.t != T_Q6_K && in.t != T_Q8_0) return -1;
        const int bv = block_values(in.t);
        if (in.ne0 % bv || in.ne0 > 16 * DEC_NT * 2 || in.nrows < 1) return -1;
        P.nb = in.ne0 / bv;
        const int body = in.t == T_Q4_K ? Q4K_BYTES : in.t == T_Q6_K ? Q6K_BODY : Q8_BODY;
        P.body_row = P.nb * body;
        const int nw = in.kind == DPH_GLU ? 2 : 1;
        const int row_bytes = nw * (P.body_row + (in.t == T_Q4_K ? 0 : 2 * P.nb));
        const int bpi = WAVE / (in.t == T_Q8_0 ? Q80::LPB : Q4K::LPB), sweeps = (P.nb + bpi - 1) / bpi;
        if (sweeps > DEC_WAVES) return -1;
        const int npass = sweeps <= 1 ? 1 : sweeps <= 2 ? 2 : sweeps <= 4 ? 4 : 8;
        P.rps = rows_per_slot(row_bytes, in.nrows, grid, DEC_WAVES / npass);
        if (!P.rps || (npass > 1 && P.rps > PART_ROWS)) return -1;
        P.nslots = (in.nrows + P.rps - 1) / P.rps;
        // A full slot: bodies plus split scales with their alignment slack.
        const int scb = in.t == T_Q4_K ? 0 : (15 + 2 * P.rps * P.nb + 15) / 16 * 16;
        if (nw * (P.rps * P.body_row + scb) > SLOT_BYTES) return -1;
        if ((int64_t)((P.nslots + grid - 1) / grid) * P.rps > YIN_MAX) return -1;
        const int64_t nblocks = (int64_t)P.nb * in.nrows;
        P.w = (const uint8_t *)in.w, P.w2 = (const uint8_t *)in.w2;
        if (in.t != T_Q4_K) {
            P.s = P.w + split_scale_offset(in.t, nblocks);
            P.s2 = P.w2 ? P.w2 + split_scale_offset(in.t, nblocks) : nullptr;
        }
    }
    std::memcpy(dst, &P, sizeof P);
    return 0;
}

hipError_t launch_decode(const DecodeIn &in, hipStream_t s) {
    const int G = in.H / in.HKV;
    const void *f = decode_kernel(in.HD, G);
    if (!f) return hipErrorInvalidValue;
    DecParams p{};
    p.ph = (CPhase *)in.phases, p.n_ph = in.n_phases;
    p.E = in.E, p.H = in.H, p.HKV = in.HKV, p.V = in.V, p.n_ctx = in.n_ctx, p.n_rot = in.n_rot, p.neox = in.neox;
    p.n_split = in.n_split, p.eps = in.eps, p.scale = in.scale;
    p.t_embd = in.t_embd, p.embd = in.embd, p.rope = (const float2 *)in.rope, p.x0 = (uint64_t *)in.x0;
    p.seq = in.seq, p.state = in.state, p.head_mode = in.head_mode, p.best = (uint64_t *)in.best;
    p.sync = (DecSync *)in.sync, p.trace = in.trace;
    p.act_off = RING_SLOTS * SLOT_BYTES;
    p.yin_off = (int)(p.act_off + act_region(in.HD, G, in.max_in));
    void *args[] = {&p};
    return hipLaunchCooperativeKernel(f, dim3(in.grid), dim3(DEC_NT), args, in.lds_bytes, s);
}

}  // namespace ts5hip
