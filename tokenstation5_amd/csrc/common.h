// Shared definitions of the HIP library: GGML block formats as they sit in
// HBM, the quantized-activation format every matvec reads, and small device
// helpers. Everything here is gfx950 (CDNA4, wave64) code.
#pragma once
#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#else
#include <hip/hip_runtime_api.h>  // host-only translation units (g++)
#endif
#include <stddef.h>
#include <stdint.h>

namespace ts5hip {

// GGML type ids (engine/src/gguf.h:12-16).
enum : uint32_t {
    T_F32 = 0, T_F16 = 1, T_Q4_0 = 2, T_Q4_1 = 3, T_Q5_0 = 6, T_Q5_1 = 7, T_Q8_0 = 8, T_Q4_K = 12, T_Q5_K = 13,
    T_Q6_K = 14
};
// The HBM layout of Q4_0, Q4_1, Q5_0, Q5_1 and Q5_K matrices (a layout id, not
// a GGML type): per 32 values 32 int8 quants q and an fp32 pair (s, m) with
// value = s * q + m, exactly the reference's unpacked value (below).
constexpr uint32_t T_Q8SM = 0x100;
__host__ __device__ inline uint32_t device_type(uint32_t t) {
    return t == T_Q4_0 || t == T_Q4_1 || t == T_Q5_0 || t == T_Q5_1 || t == T_Q5_K ? T_Q8SM : t;
}
// KvType (engine/src/backend.h:13).
enum : int { KV_F32 = 0, KV_F16 = 1, KV_Q8 = 2 };

constexpr int WAVE = 64;

__host__ __device__ constexpr inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// ---------------------------------------------------------------------------
// Weight layouts in HBM (per tensor of ne1 rows of ne0 values, row-major).
//
//  Q4_K  unchanged GGUF bytes, 144 B per 256 values: d, dmin (f16), 12 bytes
//        of packed 6-bit scales/mins, 128 bytes of nibbles. 144 = 9 x 16, so
//        every block starts on a 16-byte boundary and loads as dwordx4.
//  Q6_K  GGUF blocks are 210 B (2-byte aligned). Split at upload into a body
//        array of 208 B per block (ql[128] qh[64] scales[16], 13 x 16 B) and
//        an f16 d array behind it, so bodies load as dwordx4.
//  Q8_0  GGUF blocks are 34 B. Split into 32 B of int8 quants per block and
//        an f16 d array behind them.
//  Q4_0, Q4_1, Q5_0, Q5_1, Q5_K (T_Q8SM): 32 B of int8 quants per 32 values,
//        then an array of fp32 (s, m) pairs, value = s * q + m. Unpacked at
//        upload with the reference's own products (engine/src/quants.cpp:
//        89-131, :157-177), each exact in fp32: Q4_0 / Q5_0 q = nibble - 8 /
//        5-bit - 16, s = d, m = -0 (adding -0 keeps every value, -0
//        included); Q4_1 / Q5_1 q = nibble / 5-bit, s = d, m = m; Q5_K per
//        32-value sub-block j q = 5-bit, s = d * sc_j, m = -(dmin * m_j), the
//        reference's d1 * q - m1. So the quants fit the Q8_0 kernels, and the
//        min is one more term per block against the activation's sum.
//  F32 / F16 unchanged.
// ---------------------------------------------------------------------------
constexpr int Q4K_BYTES = 144;
constexpr int Q6K_BODY = 208;
constexpr int Q8_BODY = 32;

__host__ __device__ inline int block_values(uint32_t t) {
    switch (t) {
    case T_Q4_K: case T_Q5_K: case T_Q6_K: return 256;
    case T_Q4_0: case T_Q4_1: case T_Q5_0: case T_Q5_1: case T_Q8_0: case T_Q8SM: return 32;
    case T_F32: case T_F16: return 1;
    }
    return 0;
}
// Bytes of one GGUF block (engine/src/gguf.cpp:34-48).
__host__ __device__ inline int gguf_block_bytes(uint32_t t) {
    switch (t) {
    case T_F32: return 4;
    case T_F16: return 2;
    case T_Q4_0: return 18;
    case T_Q4_1: return 20;
    case T_Q5_0: return 22;
    case T_Q5_1: return 24;
    case T_Q8_0: return 34;
    case T_Q4_K: return 144;
    case T_Q5_K: return 176;
    case T_Q6_K: return 210;
    }
    return 0;
}
// Layouts with their quants and their scales in two arrays.
__host__ __device__ inline bool split_layout(uint32_t t) { return t == T_Q6_K || t == T_Q8_0 || t == T_Q8SM; }
// Bytes of a block's scales in a split layout.
__host__ __device__ inline int split_scale_bytes(uint32_t t) { return t == T_Q8SM ? 8 : 2; }
// Offset of the scale array of a split layout of nblocks blocks.
__host__ __device__ inline size_t split_scale_offset(uint32_t t, int64_t nblocks) {
    return align_up((size_t)nblocks * (t == T_Q6_K ? Q6K_BODY : Q8_BODY), 256);
}
// Bytes of a tensor (of GGML type or layout t) in its HBM layout; 0 if unsupported.
__host__ __device__ inline size_t device_bytes(uint32_t t, int64_t ne0, int64_t ne1) {
    const int bv = block_values(t);
    if (bv == 0 || ne0 % bv) return 0;
    const uint32_t dt = device_type(t);
    const int64_t nb = ne0 / block_values(dt) * ne1;
    if (split_layout(dt)) return split_scale_offset(dt, nb) + align_up((size_t)nb * split_scale_bytes(dt), 256);
    return (size_t)nb * gguf_block_bytes(dt);
}

// ---------------------------------------------------------------------------
// Quantized activations ("act"): the form in which every matvec reads its
// input vector x of n values (n a multiple of 32). Per 32-value sub-block s:
//   scale[s] = max|x| / XQ_MAX, X = rint(x / scale[s]) in [-XQ_MAX, XQ_MAX]
//   (XQ_MAX = 2^22 - 1: 23 significant bits, the precision of the fp32
//   input itself), X = 65536 * hi + 256 * mid + lo with lo, mid in
//   [-128, 127] and hi in [-64, 64] (the one base-256 expansion with such
//   digits),
//   sum[s] = sum of x over the sub-block (fp32, the unquantized values),
// and per 16-value run r: isum[r] = sum of X over the run (exact, int32).
// The three int8 planes feed v_dot4_i32_i8 directly against int8/uint4
// weights: sum(q * X) = 65536 dot4(q, hi) + 256 dot4(q, mid) + dot4(q, lo),
// each dot exact in int32. The rounding error per value is at most 1/2^23
// of the sub-block's largest magnitude, so a dot product over n values keeps
// a relative error of a few 1e-7 whatever the signs of its terms.
// ---------------------------------------------------------------------------
constexpr int XQ_MAX = (1 << 22) - 1;

struct Act {
    int8_t *hi, *mid, *lo;
    float *scale, *sum;
    int32_t *isum;
};
struct CAct {
    const int8_t *hi, *mid, *lo;
    const float *scale, *sum;
    const int32_t *isum;
};

__host__ __device__ inline size_t act_bytes(int64_t n) {
    return 3 * align_up((size_t)n, 256) + 2 * align_up((size_t)n / 32 * 4, 256) + align_up((size_t)n / 16 * 4, 256);
}
// The matrix-core matmuls' activation for Q4_K / Q6_K rows (n a multiple of
// 256): the same X = 65536 hi + 256 mid + lo values, scales and sums as Act,
// ordered per 256-value block so that a lane feeding k-group kq of the MFMA
// finds its 8 bytes of all 8 chunks side by side:
//   hi[4][8][8]   k-group kq, chunk c, the chunk's bytes 8 kq .. 8 kq + 7
//   mid[4][8][8]
//   lo[4][8][8]
//   scale[8], sum[8] (f32 per chunk), isum[16] (i32 per 16 values)
// 896 bytes a block.
constexpr int MACT_BLOCK = 896;
constexpr int MACT_MID = 256, MACT_LO = 512, MACT_SCALE = 768, MACT_SUM = 800, MACT_ISUM = 832;
__host__ __device__ inline size_t mact_bytes(int64_t n) { return align_up((size_t)(n / 256) * MACT_BLOCK, 256); }
// The prompt matmuls' activation (Q4_K rows, batches past 16 tokens; n a
// multiple of 256): each token's values scaled by a power of two, 2^-e, that
// puts the largest in [2^13, 2^14), then split into two fp16 planes,
// x 2^-e = hi + lo to about 22 bits:
//   per 256-value block: hi[256] f16, lo[256] f16     (1 KB)
//   then per 64-value quarter of a block, the sums X of its two 32-value
//   chunks (of x 2^-e, divided by 32) as fp16 hi + lo: (hi_0, hi_1) (lo_0, lo_1)
//   (8 bytes), then 2^e (f32).
__host__ __device__ inline size_t hact_x(int64_t n) { return (size_t)(n / 256) * 1024; }
__host__ __device__ inline size_t hact_unscale(int64_t n) { return hact_x(n) + (size_t)(n / 32) * 4; }
__host__ __device__ inline size_t hact_bytes(int64_t n) { return align_up(hact_unscale(n) + 4, 256); }

__host__ __device__ inline Act act_view(void *base, int64_t n) {
    uint8_t *p = (uint8_t *)base;
    Act a;
    a.hi = (int8_t *)p;
    p += align_up((size_t)n, 256);
    a.mid = (int8_t *)p;
    p += align_up((size_t)n, 256);
    a.lo = (int8_t *)p;
    p += align_up((size_t)n, 256);
    a.scale = (float *)p;
    p += align_up((size_t)n / 32 * 4, 256);
    a.sum = (float *)p;
    p += align_up((size_t)n / 32 * 4, 256);
    a.isum = (int32_t *)p;
    return a;
}
__host__ __device__ inline CAct cact_view(const void *base, int64_t n) {
    Act a = act_view(const_cast<void *>(base), n);
    return CAct{a.hi, a.mid, a.lo, a.scale, a.sum, a.isum};
}

// Split-K decode attention partials: per (query, key split, KV head) a group
// of G records [HD values, m, l], padded to whole 128-byte lines so that no
// line holds records of two groups (each group is handed to its merging
// workgroup on its own).
__host__ __device__ constexpr inline size_t attn_group_floats(int G, int HD) {
    return align_up((size_t)G * (HD + 2), 32);
}

#if defined(__HIPCC__)
// ---------------------------------------------------------------------------
// Device helpers.
// ---------------------------------------------------------------------------
// f16 bits to fp32: v_cvt_f32_f16 is exact for every half, subnormals
// included (f16 denormals are not flushed on gfx9).
__device__ inline float h2f(uint32_t bits16) {
    _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)bits16);
    return (float)h;
}
// fp32 to f16 bits, round to nearest even (v_cvt_f16_f32).
__device__ inline uint16_t f2h(float f) {
    _Float16 h = (_Float16)f;
    return __builtin_bit_cast(uint16_t, h);
}

__device__ inline int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }


// Cross-workgroup data. A store another workgroup will read goes out
// device-coherent (global_store ... sc1, written through past this XCD's L2);
// the writer waits for its stores (s_waitcnt vmcnt(0): __syncthreads does not
// on gfx950) before signalling, with a relaxed atomic, that they are done.
// The reader loads them device-coherent too (ld_dev). Each XCD has its own L2,
// and the L2s are not coherent with one another: an ordinary load that reads
// part of a 128-byte line could leave a copy of the whole line in this XCD's
// L2, and a later ordinary load of another part of it, written since by a
// workgroup on another XCD, would hit that stale copy. Buffers handed over
// this way are also laid out so that no 128-byte line holds data of two
// different hand-offs. None of this needs buffer_wbl2 / buffer_inv, which
// __threadfence() would emit.
// The gated unit's value: act(g) * u with SiLU (engine/src/cpu_backend.cpp:260-261), or with
// gelu the tanh form of GELU (Gemma 3, cpu_backend.cpp:71-73, :258-259).
__device__ inline float glu_act(float g, float u, int gelu) {
    if (gelu) return 0.5f * g * (1.0f + tanhf(0.7978845608f * (g + 0.044715f * g * g * g))) * u;
    return g / (1.0f + expf(-g)) * u;
}

__device__ inline void st_dev(float *p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline void st_dev(int *p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ inline float ld_dev(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ inline void wait_stores() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)
// s_waitcnt vmcnt(N) alone (gfx9 encoding: vmcnt in bits 3:0 and 15:14), as a
// builtin whose count the compiler's own wait placement takes into account.
template <int N>
__device__ inline void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

template <typename T>
__device__ inline T wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}
// Sum over the wave in registers: DPP steps (quad swaps, half-row and row
// mirrors, then the row broadcasts of lanes 15 and 31) leave the total in lane
// 63, which is read out to every lane. Six VALU ops, where a butterfly of
// __shfl_xor is six dependent LDS-crossbar round trips.
template <int CTRL, int ROW_MASK, bool BOUND>
__device__ inline float dpp_add(float x) {
    return x + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, ROW_MASK, 0xF, BOUND));
}
__device__ inline float wave_sum_dpp(float v) {
    v = dpp_add<0xB1, 0xF, true>(v);    // quad_perm [1,0,3,2]
    v = dpp_add<0x4E, 0xF, true>(v);    // quad_perm [2,3,0,1]
    v = dpp_add<0x141, 0xF, true>(v);   // row_half_mirror: 8-lane sums
    v = dpp_add<0x140, 0xF, true>(v);   // row_mirror: 16-lane sums
    v = dpp_add<0x142, 0xA, false>(v);  // row_bcast:15 into rows 1 and 3
    v = dpp_add<0x143, 0xC, false>(v);  // row_bcast:31 into rows 2 and 3
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// The sum over each 16-lane row of the wave, in every lane of the row (the
// first four steps of wave_sum_dpp).
__device__ inline float row_sum_dpp(float v) {
    v = dpp_add<0xB1, 0xF, true>(v);
    v = dpp_add<0x4E, 0xF, true>(v);
    v = dpp_add<0x141, 0xF, true>(v);
    return dpp_add<0x140, 0xF, true>(v);
}
// Max over the wave by the same DPP steps (disabled rows keep their own value).
template <int CTRL, int ROW_MASK, bool BOUND>
__device__ inline float dpp_max(float x) {
    return fmaxf(x, __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(x), __float_as_int(x), CTRL, ROW_MASK,
                                                               0xF, BOUND)));
}
__device__ inline float wave_max_dpp(float v) {
    v = dpp_max<0xB1, 0xF, true>(v);
    v = dpp_max<0x4E, 0xF, true>(v);
    v = dpp_max<0x141, 0xF, true>(v);
    v = dpp_max<0x140, 0xF, true>(v);
    v = dpp_max<0x142, 0xA, false>(v);
    v = dpp_max<0x143, 0xC, false>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
// v + the value of lane i ^ 16 (v_permlane16_swap), of lane i ^ 32
// (v_permlane32_swap): VALU lane exchanges across 16-lane rows and wave halves.
__device__ inline float add_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float add_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float max_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

// The 6-bit scale and min of sub-block j (0..7) of a K-quant block, from its
// 12 packed bytes held as three little-endian dwords a (bytes 0-3),
// b (4-7), c (8-11): sub-blocks 0-3 keep theirs in the low 6 bits of bytes j
// and j+4; 4-7 take their low 4 bits from byte j+4's low/high nibble and
// their top 2 bits from the top of bytes j-4 and j
// (engine/src/quants.cpp:64-72).
__device__ inline void kq_scale_min(int j, uint32_t a, uint32_t b, uint32_t c, int &sc, int &m) {
    if (j < 4) {
        sc = (a >> (8 * j)) & 63;
        m = (b >> (8 * j)) & 63;
    } else {
        const int s = 8 * (j - 4);
        sc = ((c >> s) & 15) | (((a >> (s + 6)) & 3) << 4);
        m = ((c >> (s + 4)) & 15) | (((b >> (s + 6)) & 3) << 4);
    }
}

// The same for the pair j = 2*sub, 2*sub + 1 that one matvec lane owns,
// without branches: bytes 2*(sub & 1) and +1 of each dword, the 6-bit form
// for sub < 2 and the split form (low 4 bits from c, top 2 from a or b) for
// sub >= 2.
__device__ inline void kq_scale_min_pair(int sub, uint32_t a, uint32_t b, uint32_t c, int &sc0, int &m0, int &sc1,
                                         int &m1) {
    const int s = 16 * (sub & 1);
    const uint32_t A = a >> s, B = b >> s, C = c >> s;
    const uint32_t split = 0u - (uint32_t)(sub >> 1);  // all ones for sub-blocks 2, 3: a bit select, no branch
    const uint32_t scw = (((C & 0x0F0Fu) | ((A >> 2) & 0x3030u)) & split) | (A & 0x3F3Fu & ~split);
    const uint32_t mw = ((((C >> 4) & 0x0F0Fu) | ((B >> 2) & 0x3030u)) & split) | (B & 0x3F3Fu & ~split);
    sc0 = (int)(scw & 0xFF), sc1 = (int)((scw >> 8) & 0xFF);
    m0 = (int)(mw & 0xFF), m1 = (int)((mw >> 8) & 0xFF);
}

// ---------------------------------------------------------------------------
// Value i of row `row` in the HBM layout of a tensor with nb blocks per row
// (bit-exact with dequantize_row).
// ---------------------------------------------------------------------------
__device__ inline float unpack_value(uint32_t t, const uint8_t *base, int64_t nblocks, int64_t row, int nb,
                                     int64_t i) {
    switch (t) {
    case T_F32:
        return ((const float *)base)[row * nb + i];
    case T_F16:
        return h2f(((const uint16_t *)base)[row * nb + i]);
    case T_Q8_0: {
        const int64_t blk = row * nb + i / 32;
        const uint16_t *ds = (const uint16_t *)(base + split_scale_offset(T_Q8_0, nblocks));
        return (float)((const int8_t *)base)[blk * Q8_BODY + (i & 31)] * h2f(ds[blk]);
    }
    case T_Q8SM: {  // s * q exact: one rounding, with or without contraction
        const int64_t blk = row * nb + i / 32;
        const float2 sm = ((const float2 *)(base + split_scale_offset(T_Q8SM, nblocks)))[blk];
        return (float)((const int8_t *)base)[blk * Q8_BODY + (i & 31)] * sm.x + sm.y;
    }
    case T_Q4_K: {
        const uint8_t *b = base + (row * nb + i / 256) * Q4K_BYTES;
        const int j = (int)(i & 255), s = j / 32, pos = j & 31;
        const uint32_t *w = (const uint32_t *)b;
        int sc, m;
        kq_scale_min(s, w[1], w[2], w[3], sc, m);
        const float d = h2f(w[0] & 0xffff), dmin = h2f(w[0] >> 16);
        const float dl = d * (float)sc, ml = dmin * (float)m;
        const uint8_t q = b[16 + 32 * (s / 2) + pos];
        const int qv = (s & 1) ? (q >> 4) : (q & 15);
        return dl * (float)qv - ml;
    }
    case T_Q6_K: {
        const int64_t blk = row * nb + i / 256;
        const uint8_t *b = base + blk * Q6K_BODY;
        const uint16_t *ds = (const uint16_t *)(base + split_scale_offset(T_Q6_K, nblocks));
        const int j = (int)(i & 255), half = j / 128, c = (j & 127) / 32, ii = j & 31;
        const uint8_t ql = b[64 * half + ii + 32 * (c & 1)];
        const uint8_t qh = b[128 + 32 * half + ii];
        const int q = (int)(((c >> 1) ? (ql >> 4) : (ql & 15)) | (((qh >> (2 * c)) & 3) << 4)) - 32;
        const int8_t sc = (int8_t)b[192 + 8 * half + ii / 16 + 2 * c];
        return h2f(ds[blk]) * (float)sc * (float)q;
    }
    }
    return 0.f;
}

// ---------------------------------------------------------------------------
// LDS DMA (global_load_lds_*): lane l's 16 (4) bytes from g land at LDS
// address lds_base + 16 l (4 l). The compiler does not see these loads:
// completion is waited for explicitly with wait_vm_n (vmcnt counts them in
// issue order with every other vector memory load).
// ---------------------------------------------------------------------------
__device__ inline void dma16(const void *g, uint32_t lds_base) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds_base) : "memory");
}
__device__ inline void dma4(const void *g, uint32_t lds_base) {
    asm volatile("global_load_lds_dword %0, off" ::"v"(g), "{m0}"(lds_base) : "memory");
}
// The same from a buffer resource at byte offset voff: offsets at or past
// the resource's size read zeros and touch no memory.
__device__ inline __amdgpu_buffer_rsrc_t buf_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, (int)bytes, 0x00020000);
}
__device__ inline void dma16b(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t lds_base) {
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds_base) : "memory");
}
// 16-run r of an activation (half r & 1 of sub-block r / 2) from its 16
// values: the three planes' bytes, the run's sum of X, and the 32-value
// chunk's scale and sum. Two threads per 32-value sub-block, in adjacent
// lanes, exchange their max and sum once (both call this together).
struct Run16 {
    uint32_t pw[3][4];  // [plane hi, mid, lo][dword] of the 16 values
    int isum;
    float scale, sum;   // of the 32-value chunk (both threads of the pair)
};
__device__ inline Run16 quant16(const float (&v)[16]) {
    Run16 q;
    float amax = 0.f, sum = 0.f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        amax = fmaxf(amax, fabsf(v[i]));
        sum += v[i];
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1, WAVE));
    sum += __shfl_xor(sum, 1, WAVE);
    const float inv = amax > 0.f ? (float)XQ_MAX / amax : 0.f;
    // The planes as bytes: with Y = X + 128 (65536 + 256 + 1), bytes 0, 1, 2
    // of Y are lo + 128, mid + 128 and hi + 128 (X = 65536 hi + 256 mid + lo
    // is the one base-256 expansion with digits in [-128, 127]; 0 < Y < 2^24
    // for |X| <= XQ_MAX), so byte permutes gather each plane of 4 values and
    // one xor with 0x80 per byte turns the offsets back into signed digits.
    constexpr int YOFF = 128 * (65536 + 256 + 1);
    int is = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        uint32_t y[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int X = max(-XQ_MAX, min(XQ_MAX, (int)rintf(v[4 * k + e] * inv)));
            y[e] = (uint32_t)(X + YOFF);
            is += X;
        }
        // t_lo: bytes 0, 1 of values 0 and 1 (or 2 and 3) interleaved, t_hi: byte 2 of each.
        const uint32_t t01 = __builtin_amdgcn_perm(y[1], y[0], 0x05010400u);
        const uint32_t t23 = __builtin_amdgcn_perm(y[3], y[2], 0x05010400u);
        const uint32_t h01 = __builtin_amdgcn_perm(y[1], y[0], 0x0C0C0602u);
        const uint32_t h23 = __builtin_amdgcn_perm(y[3], y[2], 0x0C0C0602u);
        q.pw[2][k] = __builtin_amdgcn_perm(t23, t01, 0x05040100u) ^ 0x80808080u;  // lo
        q.pw[1][k] = __builtin_amdgcn_perm(t23, t01, 0x07060302u) ^ 0x80808080u;  // mid
        q.pw[0][k] = __builtin_amdgcn_perm(h23, h01, 0x05040100u) ^ 0x80808080u;  // hi
    }
    q.isum = is, q.scale = amax / (float)XQ_MAX, q.sum = sum;
    return q;
}
// Run r into the matmul layout at `m` (the token's MAct): block r / 16, chunk
// (r % 16) / 2, bytes 16 (r & 1) .. +15 of the chunk, i.e. k-groups
// 2 (r & 1) and 2 (r & 1) + 1, in each plane.
__device__ inline void quant_run_m(const float (&v)[16], int r, uint8_t *m) {
    const Run16 q = quant16(v);
    uint8_t *blk = m + (size_t)(r / 16) * MACT_BLOCK;
    const int c = (r % 16) / 2, kq = 2 * (r & 1);
    const int plane[3] = {0, MACT_MID, MACT_LO};
#pragma unroll
    for (int P = 0; P < 3; P++) {
        *(uint2 *)(blk + plane[P] + kq * 64 + 8 * c) = make_uint2(q.pw[P][0], q.pw[P][1]);
        *(uint2 *)(blk + plane[P] + (kq + 1) * 64 + 8 * c) = make_uint2(q.pw[P][2], q.pw[P][3]);
    }
    ((int *)(blk + MACT_ISUM))[r % 16] = q.isum;
    if ((r & 1) == 0) {
        ((float *)(blk + MACT_SCALE))[c] = q.scale;
        ((float *)(blk + MACT_SUM))[c] = q.sum;
    }
}

template <int N>
__device__ inline void wait_vm_n() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
__device__ inline uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

#endif  // __HIPCC__

}  // namespace ts5hip
