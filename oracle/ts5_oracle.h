/* TEST INFRASTRUCTURE ONLY.
 *
 * A CPU restatement of ts5's fp32 reference path (engine/src/quants.cpp,
 * engine/src/cpu_backend.cpp, engine/src/engine.cpp Engine::sample). It is the
 * checker the HIP library is compared with. Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg may load it; the product never does.
 *
 * Every function is written to do the same floating-point operations in the
 * same order as the reference function it cites, so that its results are
 * bit-identical to the reference's own compiled code (checked against
 * oracle/_ref and the committed golden fixtures under tests/golden/).
 */
#pragma once
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (engine/src/gguf.h:12-16). */
enum {
    TS5O_F32 = 0, TS5O_F16 = 1, TS5O_Q4_0 = 2, TS5O_Q4_1 = 3, TS5O_Q5_0 = 6, TS5O_Q5_1 = 7,
    TS5O_Q8_0 = 8, TS5O_Q4_K = 12, TS5O_Q5_K = 13, TS5O_Q6_K = 14, TS5O_BF16 = 30
};
/* KvType (engine/src/backend.h:13). */
enum { TS5O_KV_F32 = 0, TS5O_KV_F16 = 1, TS5O_KV_Q8 = 2 };

/* fp16 <-> fp32, engine/src/quants.cpp:10-56. */
float ts5o_fp16_to_fp32(uint16_t h);
uint16_t ts5o_fp32_to_fp16(float f);

/* Values and bytes per block (engine/src/gguf.cpp:25-48); 0 if unsupported. */
int ts5o_block_values(uint32_t type);
int ts5o_block_bytes(uint32_t type);

/* dequantize_row, engine/src/quants.cpp:74-205. Returns 0, or -1 for an
 * unsupported type (the reference throws). */
int ts5o_dequantize_row(uint32_t type, const void *src, float *dst, int64_t n);

/* CPU matmul, engine/src/cpu_backend.cpp:18-37: Y[t*ystride + r] =
 * (float) sum_i (double)deq(W[r])[i] * X[t*n_in + i], rows striped over
 * `threads` threads (<= 0: hardware_concurrency). */
int ts5o_matmul(uint32_t type, const void *W, int64_t row_bytes, int64_t n_in, int64_t n_out, const float *X,
                int n, float *Y, int64_t ystride, int threads);

/* engine/src/cpu_backend.cpp:48-53, in place. */
void ts5o_rmsnorm(float *x, const float *w, int n, float eps);
/* engine/src/cpu_backend.cpp:57-68, in place; freqs may be null. */
void ts5o_rope(float *v, int n_rot, int pos, float base, int neox, const float *freqs, float scale);
/* The angle's cosine and sine exactly as the CPU rope computes them. */
void ts5o_rope_cs(int n_rot, int pos, float base, const float *freqs, float scale, float *cos_out, float *sin_out);
/* engine/src/cpu_backend.cpp:78-90, in place. */
void ts5o_round_kv(int kv_type, float *v, int n);
/* One query token's attention over positions lo..pos of an fp32 cache laid out
 * [pos][n_head_kv*head_dim]: engine/src/cpu_backend.cpp:222-248. q: [n_head*head_dim],
 * out: [n_head*head_dim]. */
void ts5o_attention(const float *q, const float *kc, const float *vc, int n_head, int n_head_kv, int head_dim,
                    int lo, int pos, float scale, float *out);
/* g = silu(g) * u, engine/src/cpu_backend.cpp:260-261. */
void ts5o_swiglu(float *g, const float *u, int64_t n);
/* g = gelu(g) * u with the tanh form of GELU, engine/src/cpu_backend.cpp:71-73, :258-259. */
void ts5o_geglu(float *g, const float *u, int64_t n);

/* Engine::sample, engine/src/engine.cpp:16-46, with its own mt19937_64. */
typedef struct ts5o_sampler ts5o_sampler;
ts5o_sampler *ts5o_sampler_new(uint64_t seed);
void ts5o_sampler_free(ts5o_sampler *s);
int32_t ts5o_sample(ts5o_sampler *s, const float *logits, int n, float temperature, float top_p, int top_k);
/* The same draw from candidates already reduced to the top k (ids and logits,
 * sorted by descending logit, ties by ascending id). */
int32_t ts5o_sample_topk(ts5o_sampler *s, const int32_t *ids, const float *logits, int k, float temperature,
                         float top_p);

/* A model, its tensors in GGUF layout (row-major, ne0 contiguous). */
typedef struct {
    int32_t n_vocab, n_embd, n_layer, n_ff, n_head, n_head_kv, head_dim, rope_dims, rope_neox;
    float rms_eps, rope_base, attn_scale, rope_scale;
    /* Gemma 3 (engine/src/model.h:28-41; zero for the other families): the embedding's
     * scale (0: none), the sliding layers' RoPE base, GELU for SiLU, and every layer but
     * each swa_pattern-th seeing only the last swa_window keys. */
    float embd_scale, rope_base_swa;
    int32_t gelu, swa_window, swa_pattern;
} ts5o_hparams;

typedef struct {
    uint32_t type;
    int64_t ne0, ne1;
    const void *data; /* null: absent */
} ts5o_tensor;

typedef struct {
    ts5o_tensor attn_norm, wq, wk, wv, wo, bq, bk, bv, q_norm, k_norm;
    ts5o_tensor ffn_norm, w_gate, w_up, w_down;
    ts5o_tensor post_attn_norm, post_ffn_norm; /* Gemma 3; absent elsewhere */
} ts5o_layer;

typedef struct ts5o_model ts5o_model;
ts5o_model *ts5o_model_new(const ts5o_hparams *hp, const ts5o_tensor *tok_embd, const ts5o_tensor *out_norm,
                           const ts5o_tensor *output, const ts5o_tensor *rope_freqs, const ts5o_layer *layers,
                           int n_ctx, int kv_type, int threads);
void ts5o_model_free(ts5o_model *m);
/* CpuBackend::forward, engine/src/cpu_backend.cpp:120-146. logits may be null
 * (fill the KV cache only). Returns 0, or -1 ("context full"). */
int ts5o_forward(ts5o_model *m, const int32_t *tokens, int n, int pos0, float *logits, int all);
/* The fp32 K (which 0) or V (which 1) cache of a layer, [n_ctx][n_head_kv*head_dim]. */
float *ts5o_kv(ts5o_model *m, int which, int layer);

#ifdef __cplusplus
}
#endif
