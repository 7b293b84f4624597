// Host-side launchers of the library's kernels (internal to libts5hip.so).
#pragma once
#include <hip/hip_runtime_api.h>
#include <stdint.h>

namespace ts5hip {

// One layer's KV cache (layout in attention.hip): q8 (k, v int8 with f16
// scales ks, vs), or f16 (k, v hold uint16 halves; ks, vs null).
struct KvLayer {
    int8_t *k;
    uint16_t *ks;
    int8_t *v;
    uint16_t *vs;
};

// quant.hip
hipError_t launch_dequant(uint32_t t, const void *w, int64_t ne0, int64_t rows, float *y, hipStream_t s);
// x[t] = row ids[*pos + t] of the embedding (pos null: ids[t]).
// scale > 0: every value times scale (Gemma 3's embedding scale).
hipError_t launch_embed(uint32_t t, const void *w, int64_t ne0, int64_t n_rows, const int32_t *ids, const int32_t *pos,
                        int ntok, float *x, hipStream_t s, float scale = 0.f);
// Split layouts (Q6_K, Q8_0): nblocks GGUF blocks in HBM -> bodies and f16 scales.
hipError_t launch_repack(uint32_t t, int64_t nblocks, const void *gguf, void *body, void *scales, hipStream_t s);
// nrows random-init rows of ne0 values (scales: the split layout's f16 array, else unused).
// n (a multiple of 32) N(0,1) values as a q8 (int8 values + f16 scale per 32) or f16 cache.
hipError_t launch_kv_synth(int64_t n, uint64_t seed, int kv_f16, void *vals, void *scales, hipStream_t s);
hipError_t launch_synth(uint32_t t, int64_t ne0, int64_t nrows, uint64_t seed, int centered, void *body, void *scales,
                        hipStream_t s);

// gemm.hip: Y[t] = W x_t for M tokens on the matrix cores; act: M records of
// act_bytes(ne0) (launch_act_quant); mode 0 store, 1 add (y = y_in + ...),
// 2 GLU (w2 = up: y = silu(W x) * (W2 x)), 2 | GLU_GELU the same with GELU's
// tanh form for SiLU (Gemma 3); y [M][ldy]; scratch:
// gemm_scratch_bytes(ne1, M, blocks per row) bytes.
constexpr int GLU_GELU = 0x10;
void set_gemm_cu_count(int n);
// gemm_wide.hip: the Q4_K prompt matmul on hact_* records (launch_gemm picks it).
int wide_splits(int64_t rows, int M, int nb, int cus, int mode);
hipError_t launch_gemm_wide(const void *w, const void *w2, int64_t ne0, int64_t ne1, const void *act, int M, int mode,
                            float *y, const float *y_in, int64_t ldy, void *scratch, int ks, hipStream_t s);
size_t gemm_scratch_bytes(int64_t rows, int M, int nb);
hipError_t launch_gemm(uint32_t t, const void *w, const void *w2, int64_t ne0, int64_t ne1, const void *act, int M,
                       int mode, float *y, const float *y_in, int64_t ldy, void *scratch, hipStream_t s);
// Q4_K, 1-5 tokens, ne0 a multiple of 256 up to 4096: the matmul with the
// activation built by each workgroup in LDS from the fp32 x [M][xstride]
// (rms-normalised by norm_w first when given): no launch_gemm_act record.
bool gemm_fused_fits(uint32_t t, int64_t ne0, int M);
// qout (optional): the outputs also as launch_gemm_act's Q4_K records for
// the next matmul (mact records of ne1 values per token, so that it needs
// no launch_gemm_act); where gemm_fused_qout_fits.
bool gemm_fused_qout_fits(int64_t ne0, int64_t ne1, int M);
hipError_t launch_gemm_fused(const void *w, const void *w2, int64_t ne0, int64_t ne1, const float *x,
                             int64_t xstride, const float *norm_w, float eps, int M, int mode, float *y,
                             const float *y_in, int64_t ldy, hipStream_t s, void *qout = nullptr);

// act.hip
hipError_t launch_rmsnorm(const float *x, const float *w, float eps, int n, int ntok, float *y, hipStream_t s);
// x_t += rmsnorm(o_t) * w for ntok tokens (Gemma 3's norms after attention and the FFN); n <= 8192.
hipError_t launch_norm_add(const float *o, int64_t ostride, const float *w, float eps, int n, int ntok, float *x,
                           int64_t xstride, hipStream_t s);
// The activation records launch_gemm reads for type t and ntok tokens
// (gemm_act_form: Act, the matmul layout mact_* or the fp16 pair form hact_*),
// gemm_act_bytes(t, n, ntok) per token.
enum { GA_ACT = 0, GA_MACT = 1, GA_HACT = 2 };
int gemm_act_form(uint32_t t, int64_t n, int ntok);
size_t gemm_act_bytes(uint32_t t, int64_t n, int ntok);
hipError_t launch_gemm_act(uint32_t t, const float *x, int64_t xstride, const float *w, float eps, int n, int ntok,
                           void *act, hipStream_t s);
hipError_t launch_act_quant(const float *x, int64_t xstride, const float *w, float eps, int n, int ntok, void *act,
                            hipStream_t s);

// matvec.hip: y (=|+=) W x for fp32 x, rms-normalised by norm_w first when given.
void set_cu_count(int n);
hipError_t launch_matvec(uint32_t t, const void *w, int64_t ne0, int64_t ne1, const float *x, const float *norm_w,
                         float eps, float *y, int add, hipStream_t s);
// y = silu(Wg x) * (Wu x); with gelu, GELU (tanh form) for SiLU.
hipError_t launch_matvec_glu(uint32_t t, const void *wg, const void *wu, int64_t ne0, int64_t ne1, const float *x,
                             const float *norm_w, float eps, float *y, hipStream_t s, int gelu = 0);
// ntok tokens (x rows xstride apart, y rows ldy apart) one matvec launch each:
// mode 0 store, 1 add, 2 gate/up + SiLU (w2 the up rows; 2 | GLU_GELU: GELU).
// F16 / F32 matrices' batches.
hipError_t launch_matvec_tokens(uint32_t t, const void *w, const void *w2, int64_t ne0, int64_t ne1, const float *x,
                                int64_t xstride, const float *norm_w, float eps, int ntok, int mode, float *y,
                                int64_t ldy, hipStream_t s);
// y = W x and out[0] = the first argmax of y; with seq: seq[*pos + 1] = it, ++*pos.
// Completion counters (a workgroup counts in; the last one to arrive does the
// epilogue) sit CTR_STRIDE ints apart: atomics from different workgroups to
// one 64-byte granule are served one after another (about 10 ns each on
// this chip; 256 of them add 1.7 us to a launch), to different lines in
// parallel.
constexpr int CTR_STRIDE = 32;
// The head's argmax counts its workgroups into ARGMAX_FAN sub-counters, the
// last arrival at each into a top counter: ARGMAX_CTR_INTS ints.
constexpr int ARGMAX_FAN = 16;
constexpr int ARGMAX_CTR_INTS = (1 + ARGMAX_FAN) * CTR_STRIDE;
// scratch: matvec_argmax_scratch_bytes(); counter: ARGMAX_CTR_INTS ints, zero
// before (and after) the launch.
size_t matvec_argmax_scratch_bytes();
hipError_t launch_matvec_argmax(uint32_t t, const void *w, int64_t ne0, int64_t ne1, const float *x,
                                const float *norm_w, float eps, float *y, void *scratch, int *counter, int32_t *out,
                                int32_t *seq, int32_t *pos, hipStream_t s);

// attention.hip
// kv_f16: the cache holds f16 values (k / v as uint16 [HKV][n_ctx][HD], no
// scales) instead of q8.
hipError_t launch_rope_kv(const float *qkv, int64_t qkv_stride, const float *bias, const float *q_norm,
                          const float *k_norm, float eps, const float *rope_cs, int n_rot, int neox,
                          const int32_t *pos0, int H, int HKV, int HD, int n_ctx, int ntok, float *q_out, KvLayer kv,
                          int kv_f16, hipStream_t s);
bool attn_supported(int H, int HKV, int HD);
// Flash decode (attention.hip: k_attn). q rows of B queries; with rope each
// row holds the token's raw q, k, v ((H + 2 HKV) HD values), and q (with
// append, B == 1, also the token's K/V) gets bias / norm / RoPE here.
// New keys a query of a batch on one cache reads from its workgroup's LDS
// (append: batches of up to this many tokens round and append their own K/V).
constexpr int ATTN_MAX_NEW = 16;
struct AttnIO {
    const float *q;
    int64_t q_stride;
    int rope, append;
    const float *bias, *q_norm, *k_norm;
    float eps;
    const float *rope_cs;
    int n_rot, neox;
    KvLayer kv;
    int kv_f16;  // the cache holds f16 values (no scales) instead of q8
    int kv_per_batch, n_ctx;
    const int32_t *n_keys;
    int B, H, HKV, HD, n_split;
    float scale;
    float *part;    // attn_partial_bytes(B, n_split, H, HKV, HD), 128-byte aligned
    int *counters;  // B * HKV * CTR_STRIDE ints, zero before the first launch (kept zero after)
    float *out;     // [B][H * HD]
    // Or null: with attn_mq_fits, the output also as the Q4_K small-batch
    // matmul's activation records of the H * HD values, act_stride bytes a
    // token (the next projection then reads them instead of quantizing).
    void *act_out;
    int64_t act_stride;
    // > 0: a sliding layer's window (Gemma 3): each query sees only its last
    // `win` keys, its own included (engine/src/cpu_backend.cpp:228-229).
    int win;
};
hipError_t launch_attn(const AttnIO &io, hipStream_t s);
// Whether launch_attn takes the batch's queries together on the matrix cores
// (one q8 cache, 2..ATTN_MAX_NEW queries, B x G <= 32, head dimension 128);
// its partials fit attn_partial_bytes(B, n_split, ...) as the per-query
// kernel's do, with the split count from attn_mq_splits.
bool attn_mq_fits(int B, int H, int HKV, int HD, int kv_f16, int kv_per_batch);
// The no-allocation entry point's scratch: a static device array of
// NOALLOC_BYTES per GPU, merge counters first (up to 4096 (query, KV head)
// pairs, CTR_STRIDE ints apart), then up to NOALLOC_BYTES -
// NOALLOC_COUNTER_BYTES of split partials. attn_noalloc_setup (once per
// device, that device current; the library's init calls it) looks up its
// address there and zeroes the counters.
constexpr size_t NOALLOC_BYTES = 4u << 20;
constexpr size_t NOALLOC_COUNTER_BYTES = (size_t)4096 * CTR_STRIDE * 4;
constexpr int NOALLOC_DEVICES = 64;
hipError_t attn_noalloc_setup(int device, void **ptr, hipStream_t s);
// attn_prefill.hip: causal attention of nq consecutive queries (positions p0..,
// rows q [nq][q_stride]) over one q8 or (kv_f16) f16 cache on the matrix cores;
// out [nq][H * HD]; part: attn_prefill_partial_bytes(nq, H, HD, p0 + nq) bytes.
bool attn_prefill_supported(int H, int HKV, int HD);
size_t attn_prefill_partial_bytes(int nq, int H, int HD, int64_t max_keys);
hipError_t launch_attn_prefill(const float *q, int64_t q_stride, KvLayer kv, int kv_f16, int n_ctx, int H, int HKV,
                               int HD, int p0, int nq, float scale, float *part, float *out, hipStream_t s);
hipError_t launch_kv_read(KvLayer kv, int which, int HKV, int HD, int n_ctx, int pos0, int n, int kv_f16, float *out,
                          hipStream_t s);
hipError_t launch_kv_write(KvLayer kv, int which, int HKV, int HD, int n_ctx, int pos0, int n, int kv_f16,
                           const float *in, hipStream_t s);

// sample.hip
size_t argmax_scratch_bytes(int rows);
// out[r] = argmax of row r; with seq (one row): seq[*pos + 1] = id, ++*pos.
hipError_t launch_argmax(const float *x, int n, int rows, void *scratch, int32_t *out, int32_t *seq, int32_t *pos,
                         hipStream_t s);
hipError_t launch_advance(int32_t *pos, hipStream_t s);
hipError_t launch_set_pos(int32_t *pos, int32_t v, hipStream_t s);
// The k (<= topk_max()) largest of each of `rows` rows of n (<= topk_max_n())
// logits, descending, ties by ascending id: vals / ids [rows][k].
size_t topk_scratch_bytes(int rows);
int topk_max();
int topk_max_n();
hipError_t launch_topk(const float *x, int n, int k, int rows, void *scratch, float *vals, int32_t *ids,
                       hipStream_t s);

}  // namespace ts5hip
