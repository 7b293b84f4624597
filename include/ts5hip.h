/* ts5hip.h: the C ABI of ts5's MI355X (gfx950) backend, libts5hip.so.
 *
 * This is the thin layer the C++ host engine calls in place of the Vulkan
 * backend (engine/src/vk_backend.cpp). Plain C types only: opaque handles,
 * pointers and sizes. Every entry point returns TS5HIP_OK (0) or a negative
 * TS5HIP_ERR_* code, with the message at ts5hip_last_error(ctx). A context
 * owns one HIP stream; calls on one context are not thread-safe (the
 * reference's Backend is not re-entrant either, engine/src/server.h:17-18).
 * The library owns device memory; callers own host buffers.
 *
 * Citations name the reference interface each entry point replaces
 * (paths under ThatRetiredDude/TokenStation5).
 */
#ifndef TS5HIP_H
#define TS5HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TS5HIP_OK 0
#define TS5HIP_ERR_ARG (-1)          /* invalid argument or shape */
#define TS5HIP_ERR_HIP (-2)          /* HIP runtime error */
#define TS5HIP_ERR_UNSUPPORTED (-3)  /* type / shape this backend has no kernel for */
#define TS5HIP_ERR_CONTEXT_FULL (-4) /* "context full" (engine/src/vk_backend.cpp:271) */
#define TS5HIP_ERR_STATE (-5)        /* missing tensor, model not complete */

/* GGML type ids (engine/src/gguf.h:12-16) with kernels here. */
enum { TS5HIP_F32 = 0, TS5HIP_F16 = 1, TS5HIP_Q8_0 = 8, TS5HIP_Q4_K = 12, TS5HIP_Q6_K = 14 };
/* KvType (engine/src/backend.h:13). Q8 and F16 caches are implemented on the GPU. */
enum { TS5HIP_KV_F32 = 0, TS5HIP_KV_F16 = 1, TS5HIP_KV_Q8 = 2 };

typedef struct ts5hip_ctx ts5hip_ctx;
typedef struct ts5hip_model ts5hip_model;
typedef struct ts5hip_sampler ts5hip_sampler;

/* ---- device and context (replaces VkContext, engine/src/vk_context.h:14-36) ---- */

/* The last error on ctx, or of the calling thread when ctx is null. */
const char *ts5hip_last_error(const ts5hip_ctx *ctx);
/* Opens HIP device `device` and a stream on it. Fails unless it is gfx950. */
int ts5hip_init(int device, ts5hip_ctx **out);
/* Destroy every model of the context first (ts5hip_model_destroy uses it). */
void ts5hip_destroy(ts5hip_ctx *ctx);
/* Compute units, the gfx architecture name, and HBM bytes of the device. */
int ts5hip_device_info(ts5hip_ctx *ctx, int *n_cu, char *arch, int arch_len, int64_t *hbm_bytes);

/* ---- device memory and timing (test and benchmark plumbing) ---- */
int ts5hip_alloc(ts5hip_ctx *ctx, size_t bytes, void **dptr);
int ts5hip_free(ts5hip_ctx *ctx, void *dptr);
int ts5hip_upload(ts5hip_ctx *ctx, void *dst, const void *src, size_t bytes);   /* host -> device, synchronous */
int ts5hip_download(ts5hip_ctx *ctx, void *dst, const void *src, size_t bytes); /* device -> host, synchronous */
int ts5hip_memset(ts5hip_ctx *ctx, void *dst, int value, size_t bytes);
int ts5hip_sync(ts5hip_ctx *ctx);
/* HIP events on the context's stream around the work enqueued between them. */
int ts5hip_timer_begin(ts5hip_ctx *ctx);
int ts5hip_timer_end(ts5hip_ctx *ctx, float *ms);
/* Event i (0..4095) recorded on the context's stream; ts5hip_timer_marks: the n - 1 intervals
 * (ms) between marks 0..n-1, after the last one completes (per-launch kernel times). */
int ts5hip_timer_mark(ts5hip_ctx *ctx, int i);
int ts5hip_timer_marks(ts5hip_ctx *ctx, int n, float *ms);

/* ---- weights (replaces VkBackend::upload_weights, engine/src/vk_backend.cpp:531-600) ---- */

/* Whether a matrix of this GGML type has GPU kernels (vk_supports_type, engine/src/backend.h:89): the
 * reference's GPU types (engine/src/vk_backend.cpp:156-170) F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0,
 * Q4_K, Q5_K, Q6_K. Q4_0, Q4_1, Q5_0, Q5_1 and Q5_K are unpacked at upload, exactly, into int8
 * quants with an fp32 (scale, min) per 32 values; F16 / F32 rows are read as they are. */
int ts5hip_supports_type(uint32_t type);
/* Bytes of a (ne1 rows x ne0 values) tensor in its HBM layout; -1 if unsupported. */
int64_t ts5hip_weight_bytes(uint32_t type, int64_t ne0, int64_t ne1);
/* GGUF bytes on the host (engine/src/model.h:44-53 Weight::data) -> HBM layout at dst. */
int ts5hip_weight_upload(ts5hip_ctx *ctx, uint32_t type, int64_t ne0, int64_t ne1, const void *gguf, void *dst);
/* n (a multiple of 32) values drawn N(0,1) into a cache layout, seeded: KV_Q8 as the q8 cache
 * rounds them (int8 values, an f16 scale per 32 consecutive values: round_kv,
 * engine/src/cpu_backend.cpp:78-90), KV_F16 as f16 values (scales unused). Benchmark inputs. */
int ts5hip_kv_synth(ts5hip_ctx *ctx, uint64_t seed, int64_t n, int kv_type, void *values, void *scales);
/* Seeded random-init weights written straight into HBM layout (benchmark inputs). */
int ts5hip_weight_synth(ts5hip_ctx *ctx, uint32_t type, int64_t ne0, int64_t ne1, uint64_t seed, int centered,
                        void *dst);

/* ---- per-op entry points: device pointers, asynchronous on the context's stream ---- */

/* dequantize_row (engine/src/quants.h:11) of `rows` rows in HBM layout -> fp32, bit-exact. */
int ts5hip_dequantize(ts5hip_ctx *ctx, uint32_t type, const void *w, int64_t ne0, int64_t rows, float *y);
/* Bytes of one token's quantized activation of n values (the matvec input form). */
int64_t ts5hip_act_bytes(int64_t n);
/* x [ntok][n] fp32 -> ntok activations; with norm_w, rmsnorm first (engine/src/cpu_backend.cpp:48-53). */
int ts5hip_act_quantize(ts5hip_ctx *ctx, const float *x, const float *norm_w, float eps, int64_t n, int ntok,
                        void *act);
/* rmsnorm (engine/src/cpu_backend.cpp:48-53): y = x / rms(x) * w per token. */
int ts5hip_rmsnorm(ts5hip_ctx *ctx, const float *x, const float *w, float eps, int64_t n, int ntok, float *y);
/* One-token matvec y (+)= W x (engine/src/cpu_backend.cpp:18-37 at n = 1; mv16_q4_k /
 * mv16_q6_k / matmul_q8_0 in engine/src/vk_backend.cpp:863-880). W: ne1 rows of ne0 in HBM
 * layout; x: ne0 fp32, rms-normalised by norm_w first when norm_w is not null (the norm
 * before every projection, engine/src/cpu_backend.cpp:193, :252). */
int ts5hip_matvec(ts5hip_ctx *ctx, uint32_t type, const void *w, int64_t ne0, int64_t ne1, const float *x,
                  const float *norm_w, float eps, float *y, int accumulate);
/* Fused gate/up + SiLU (mv16_glu_q4_k, engine/src/vk_backend.cpp:1009-1021; CPU
 * engine/src/cpu_backend.cpp:253-261): y = silu(Wg x') * (Wu x'), x' = x or rmsnorm(x). */
int ts5hip_matvec_glu(ts5hip_ctx *ctx, uint32_t type, const void *w_gate, const void *w_up, int64_t ne0,
                      int64_t ne1, const float *x, const float *norm_w, float eps, float *y);
/* The output head and the greedy pick in one pass (engine/src/cpu_backend.cpp:270-285 then
 * engine/src/engine.cpp:17): y = W x' and out_dev[0] = the first index of max(y). */
int ts5hip_matvec_argmax(ts5hip_ctx *ctx, uint32_t type, const void *w, int64_t ne0, int64_t ne1, const float *x,
                         const float *norm_w, float eps, float *y, int32_t *out_dev);
/* The projections of ntok tokens at once, each weight read once per call
 * (engine/src/cpu_backend.cpp:18-41 at n > 1; the reference's GPU path uses mvt_q4_k / mvt_q6_k
 * for 2..8 tokens and matmul_big for prompts, engine/src/vk_backend.cpp:835-918):
 * y[t] (+)= W x'_t for t < ntok (1..4096), x' = x_t or rmsnorm(x_t) by norm_w.
 * x: [ntok][ne0] fp32, y: [ntok][ne1] fp32. Matrix cores; the numerics of ts5hip_matvec. */
int ts5hip_matmul(ts5hip_ctx *ctx, uint32_t type, const void *w, int64_t ne0, int64_t ne1, const float *x, int ntok,
                  const float *norm_w, float eps, float *y, int accumulate);
/* The same for gate/up + SiLU (engine/src/cpu_backend.cpp:253-261): y[t] = silu(Wg x'_t) * (Wu x'_t). */
int ts5hip_matmul_glu(ts5hip_ctx *ctx, uint32_t type, const void *w_gate, const void *w_up, int64_t ne0,
                      int64_t ne1, const float *x, int ntok, const float *norm_w, float eps, float *y);
/* RoPE angles as engine/src/cpu_backend.cpp:59-61 computes them, for positions
 * [0, n_pos): dst gets [n_pos][n_rot/2] (cos, sin) float pairs. freqs: n_rot/2 divisors or null. */
int ts5hip_rope_table(ts5hip_ctx *ctx, int n_rot, int n_pos, float base, float scale, const float *freqs_host,
                      float *dst);
/* The q/k/v rows of ntok tokens at positions *pos0_dev.. (qkv: [ntok][(H + 2 HKV) HD]):
 * bias, optional per-head norm, RoPE, then K and V rounded to q8 and stored at their slots
 * (qkv_post_q8, engine/src/vk_backend.cpp:1145-1164; round_kv, engine/src/cpu_backend.cpp:78-90).
 * Cache: k8/v8 int8 [n_head_kv][n_ctx][head_dim], ks/vs f16 [n_head_kv][n_ctx][head_dim/32].
 * q_out: [ntok][H HD] fp32. bias ([(H + 2 HKV) HD]), q_norm, k_norm ([HD]) may be null. */
int ts5hip_rope_kv_append(ts5hip_ctx *ctx, const float *qkv, int ntok, const int32_t *pos0_dev, int n_head,
                          int n_head_kv, int head_dim, int n_rot, int neox, const float *rope_cs, int n_ctx,
                          const float *bias, const float *q_norm, const float *k_norm, float eps, float *q_out,
                          void *k8, void *ks, void *v8, void *vs);
/* Split-K flash decode over the q8 cache (attn_q8 + attn_merge, engine/src/vk_backend.cpp:937-995;
 * CPU engine/src/cpu_backend.cpp:222-248). q: [B][H HD]. kv_per_batch = 1: query b reads
 * sequence b's cache (B caches of n_ctx slots back to back) over n_keys_dev[b] keys;
 * kv_per_batch = 0: one cache, query b reads n_keys_dev[0] + b + 1 keys (n_keys_dev[0] =
 * the batch's first position). out: [B][H HD] fp32. n_split <= 0 picks a split count that
 * fills the GPU. */
int ts5hip_attn_decode(ts5hip_ctx *ctx, const float *q, int B, int n_head, int n_head_kv, int head_dim,
                       const void *k8, const void *ks, const void *v8, const void *vs, int n_ctx,
                       const int32_t *n_keys_dev, int kv_per_batch, float scale, int n_split, float *out);
/* ts5hip_attn_decode over an f16 cache (KvType::F16, engine/src/backend.h:13; the reference's
 * long-context attn_dec, engine/shaders/attn_dec.glsl, policy engine/src/vk_backend.cpp:958-960):
 * k16 / v16 hold f16 values [n_head_kv][n_ctx][head_dim] (or B such caches with kv_per_batch),
 * no scales; otherwise as ts5hip_attn_decode. */
int ts5hip_attn_decode_f16(ts5hip_ctx *ctx, const float *q, int B, int n_head, int n_head_kv, int head_dim,
                           const void *k16, const void *v16, int n_ctx, const int32_t *n_keys_dev, int kv_per_batch,
                           float scale, int n_split, float *out);
/* ts5hip_attn_decode without any allocation: no counterpart in the reference. For callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). The same arguments, kernels and results as
 * ts5hip_attn_decode, but the split partials and merge counters live in a static device array
 * of 4 MiB per GPU (held until the process ends; its address is looked up at ts5hip_init):
 * calls needing more than 3.5 MiB of partials (B x n_split x n_head_kv x ~2 KB at head_dim
 * 128) fail with TS5HIP_ERR_ARG. Every call on one GPU shares that array, whichever context
 * makes it: calls that overlap on one GPU (other streams, other contexts, other threads) race. */
int ts5hip_attn_decode_noalloc(ts5hip_ctx *ctx, const float *q, int B, int n_head, int n_head_kv, int head_dim,
                               const void *k8, const void *ks, const void *v8, const void *vs, int n_ctx,
                               const int32_t *n_keys_dev, int kv_per_batch, float scale, int n_split, float *out);
/* Causal prompt attention on the matrix cores (attn_pf, engine/shaders/attn_pf.glsl with its
 * policy at engine/src/vk_backend.cpp:954-961; CPU engine/src/cpu_backend.cpp:222-248): nq
 * queries at positions pos0 .. pos0 + nq - 1 over one q8 cache (the layout above), query t
 * reading keys 0 .. pos0 + t. q: [nq][H HD]; out: [nq][H HD] fp32. head_dim 64 or 128 and
 * n_head / n_head_kv at most 64; otherwise TS5HIP_ERR_UNSUPPORTED. */
int ts5hip_attn_prompt(ts5hip_ctx *ctx, const float *q, int nq, int n_head, int n_head_kv, int head_dim,
                       const void *k8, const void *ks, const void *v8, const void *vs, int n_ctx, int pos0,
                       float scale, float *out);
/* The same over an f16 cache (KvType::F16: k16 / v16 the halves, [n_head_kv][n_ctx][head_dim],
 * no scales), the reference's attn_pf128 for f16 caches (engine/shaders/attn_pf128.comp over
 * attn_pf.glsl; chosen at engine/src/vk_backend.cpp:954-975). */
int ts5hip_attn_prompt_f16(ts5hip_ctx *ctx, const float *q, int nq, int n_head, int n_head_kv, int head_dim,
                           const void *k16, const void *v16, int n_ctx, int pos0, float scale, float *out);
/* Greedy token per row: the first maximum of each row of n logits (engine/src/engine.cpp:17). */
int ts5hip_argmax(ts5hip_ctx *ctx, const float *x, int n, int rows, int32_t *out_dev);
/* The k (<= 64) largest of n logits, descending, ties by ascending id (the candidate set
 * of engine/src/engine.cpp:19-33). */
int ts5hip_topk(ts5hip_ctx *ctx, const float *x, int n, int k, float *vals_dev, int32_t *ids_dev);

/* ---- the sampler: Engine::sample (engine/src/engine.cpp:16-46) on host, std::mt19937_64 ---- */
ts5hip_sampler *ts5hip_sampler_new(uint64_t seed);
void ts5hip_sampler_free(ts5hip_sampler *s);
/* Draw from candidates sorted by descending logit: weights exp((l - l0) / T) in double, the
 * shortest prefix reaching top_p, std::discrete_distribution. */
int32_t ts5hip_sampler_draw(ts5hip_sampler *s, const int32_t *ids, const float *logits, int k, float temperature,
                            float top_p);

/* ---- model: Backend (engine/src/backend.h:16-44) over HIP ---- */

/* HParams (engine/src/model.h:14-42), the fields the token loop reads. The last five are
 * Gemma 3's (model.h:28-41, set by engine/src/model.cpp:44-63; zero for the other families):
 * the embedding's scale (0: none), the RoPE base of the sliding layers (which also skip
 * rope_scale), GELU (tanh form) for SiLU, and every layer l with l % swa_pattern <
 * swa_pattern - 1 seeing only the last swa_window keys. Layers with post_attention_norm /
 * post_ffw_norm tensors normalize their attention / FFN output before the residual add.
 * Every layer keeps a full cache here (the 288 GB of HBM hold the training context of every
 * Gemma 3 size), so rewind_limit stays unlimited. */
typedef struct {
    int32_t n_vocab, n_embd, n_layer, n_ff, n_head, n_head_kv, head_dim, rope_dims, rope_neox;
    float rms_eps, rope_base, attn_scale, rope_scale;
    float embd_scale, rope_base_swa;
    int32_t gelu, swa_window, swa_pattern;
} ts5hip_hparams;

/* make_vk_backend (engine/src/backend.h:82) for HIP: a model of these hyperparameters with a
 * KV cache of n_ctx positions. Tensors are then set by GGUF name (engine/src/model.cpp:89-119). */
int ts5hip_model_create(ts5hip_ctx *ctx, const ts5hip_hparams *hp, int n_ctx, int kv_type, ts5hip_model **out);
void ts5hip_model_destroy(ts5hip_model *m);
/* A tensor from its GGUF bytes on the host. */
int ts5hip_model_set_tensor(ts5hip_model *m, const char *name, uint32_t type, int64_t ne0, int64_t ne1,
                            const void *gguf);
/* Rows [row0, row0 + nrows) of a tensor of ne1 rows from their GGUF bytes (a loader streaming
 * a file through a bounded buffer; vectors are set whole). The tensor counts as set once its
 * last rows are. */
int ts5hip_model_set_tensor_rows(ts5hip_model *m, const char *name, uint32_t type, int64_t ne0, int64_t ne1,
                                 int64_t row0, int64_t nrows, const void *gguf);
/* A tensor generated in HBM (ts5hip_weight_synth). */
int ts5hip_model_synth_tensor(ts5hip_model *m, const char *name, uint32_t type, int64_t ne0, int64_t ne1,
                              uint64_t seed, int centered);
/* Backend::forward (engine/src/backend.h:21-24): tokens at positions pos0..pos0+n-1; logits of
 * the last token, or of all n when all_logits, into logits ([n or 1][n_vocab]); logits null:
 * fill the KV cache only. */
int ts5hip_forward(ts5hip_model *m, const int32_t *tokens, int n, int pos0, float *logits, int all_logits);
/* Backend::forward_in_place / logits_view (engine/src/backend.h:25-33): the logits rows stay
 * in HBM; ts5hip_logits_view copies them to pinned host memory on its first call after a
 * forward (room for 256 rows) and returns that copy. */
int ts5hip_forward_in_place(ts5hip_model *m, const int32_t *tokens, int n, int pos0, int all_logits);
const float *ts5hip_logits_view(const ts5hip_model *m);
/* Backend::n_ctx / kv_type (engine/src/backend.h:34-39). */
int ts5hip_n_ctx(const ts5hip_model *m);
int ts5hip_kv_type(const ts5hip_model *m);
/* How single-token steps and verify batches (2-16 tokens, one graph per token count and
 * logits rows, captured on first use) run once every tensor is set: 1 HIP graph replays, 0
 * direct kernel launches (TS5HIP_GRAPHS=0 at model creation); < 0 an error. No counterpart in
 * the reference (its Vulkan backend has one path): for tests and profiles. */
int ts5hip_token_path(ts5hip_model *m);
/* The k (1..64) largest logits of rows [row0, row0 + nrows) of the last forward, found on the
 * GPU where the rows stay, descending with ties by ascending id, into host arrays
 * vals/ids [nrows][k]. k = 1 is the greedy pick of engine/src/engine.cpp:17. This is the
 * additive Backend::topk_view hook that lets Engine::sample (engine/src/engine.cpp:16-46) and
 * the draft model's greedy step (engine/src/engine.cpp:124) read k candidates per row
 * instead of n_vocab floats; the logits rows reach the host only if ts5hip_logits_view is
 * called. */
int ts5hip_logits_topk(ts5hip_model *m, int row0, int nrows, int k, float *vals, int32_t *ids);
/* Engine::sample (engine/src/engine.cpp:16-46) of row `row` of the last forward: the GPU
 * argmax (temperature <= 0) or top-k candidates and the host draw; the whole row is read on
 * the host only when ties or a top_k past 63 leave the candidates short of deciding it. */
int32_t ts5hip_model_sample(ts5hip_model *m, ts5hip_sampler *s, int row, float temperature, float top_p,
                            int top_k);
/* Greedy decode kept on the device (run_bench's generation loop, engine/src/checks.cpp:195-199,
 * with argmax feedback): `token` at `pos`, then n_steps tokens, each the argmax of the previous
 * step's logits; ids_out gets those n_steps ids. One HIP graph replay per token. */
int ts5hip_generate_greedy(ts5hip_model *m, int32_t token, int pos, int n_steps, int32_t *ids_out);
/* K (which 0) or V (1) of `layer` at positions [pos0, pos0+n), dequantized to fp32
 * [n][n_head_kv * head_dim] (the CPU cache's layout, engine/src/cpu_backend.cpp:95-97). */
int ts5hip_kv_read(ts5hip_model *m, int layer, int which, int pos0, int n, float *out);
/* The reverse of ts5hip_kv_read, for tests: fp32 K (which 0) or V (1) values [n][n_head_kv *
 * head_dim] stored at positions [pos0, pos0 + n) of `layer`, rounded as the cache keeps them (q8 as
 * round_kv, engine/src/cpu_backend.cpp:78-90, or f16): values already so rounded are stored
 * exactly. No counterpart in the reference (its Backend exposes no cache). */
int ts5hip_kv_write(ts5hip_model *m, int layer, int which, int pos0, int n, const float *in);
/* Backend::take_profile (engine/src/backend.h:40-43): text since the last call. With TS5_PROFILE
 * (or TS5HIP_PROFILE) set when the model is made: GPU time of its forward calls; with the value 1
 * also GPU time per kernel and weight role ("matvec_q4_k ffn_down", "attention_q8 decode", ...),
 * most first, with share and launch count (the reference's per-dispatch timestamps,
 * engine/src/vk_backend.cpp:347-358, :737-749, :926-932). Graph replays (single tokens, verify
 * batches) then carry an event node after each kernel and are read after every replay (a host
 * wait per replay; each kernel's time includes its node's, a few us); with TS5HIP_GRAPHS=0 every
 * launch runs directly with an event after it. A buffer too small is an error that keeps the
 * profile. */
int ts5hip_take_profile(ts5hip_model *m, char *buf, int len);

/* ---- GGUF files, KV sizing (engine/src/backend.h:53-81, engine/src/model.cpp:13-138,
 * engine/src/vk_backend.cpp:531-600, :620-648, :1364-1402) ---- */

/* kv_bytes_per_token (engine/src/backend.h:56): bytes of K and V per token of context over all
 * layers in a cache of kv_type (q8: a byte per value and an f16 scale per 32). */
uint64_t ts5hip_kv_bytes_per_token(const ts5hip_hparams *hp, int kv_type);
/* fit_context (engine/src/backend.h:72): the context that fits in `memory` beside `used` bytes and
 * 1 GiB kept for everything else, a multiple of 1024 up to cap; 0 if not even 1024 tokens fit. */
int ts5hip_fit_context(uint64_t memory, uint64_t used, uint64_t per_token, int cap);
/* f16_reaches (engine/src/backend.h:76): whether an f16 context of f16_ctx tokens is the whole
 * training context (then a q8 request gets an f16 cache). */
int ts5hip_f16_reaches(int f16_ctx, int train);
/* The hyperparameters of a GGUF file as Model::open derives them (engine/src/model.cpp:13-68; llama,
 * mistral, qwen2, qwen3), its training context, and the HBM bytes the model takes beside its KV
 * cache (weights in their HBM layouts, activations, scratch). */
int ts5hip_gguf_hparams(const char *path, ts5hip_hparams *hp, int *n_ctx_train, int64_t *fixed_bytes);
/* make_vk_backend(Model&, path, n_ctx, device, err) for HIP with the file included
 * (engine/src/backend.h:82; Model::open + load, engine/src/model.cpp:13-138; the weight upload,
 * engine/src/vk_backend.cpp:531-600): the model of a GGUF file with a cache of n_ctx positions,
 * its tensors read by `threads` workers (<= 0: 4) with pread into pinned buffers while earlier
 * slices go to HBM. n_ctx 0: the context that fits the device's free memory, at most the training
 * context (engine/src/vk_backend.cpp:620-648), and a q8 request gets an f16 cache when f16
 * reaches the training context. kv_type_out (may be null): the cache type chosen. */
int ts5hip_model_load(ts5hip_ctx *ctx, const char *path, int n_ctx, int kv_type, int threads, ts5hip_model **out,
                      int *kv_type_out);

/* ---- ts5 check (engine/src/checks.h, engine/src/checks.cpp:22-160) ---- */

/* CheckResult (engine/src/checks.h:17-24). */
typedef struct {
    int32_t n, same_top, worst; /* worst: the position of max_diff */
    double max_diff, rel, gpu_ms;
    int32_t pass, saved; /* saved: the reference logits came from a .ts5ref file */
} ts5hip_check_result;
/* The check's n test tokens (engine/src/checks.cpp:22-26): 1000 + (i * 7919) % (n_vocab - 1000). */
int ts5hip_check_tokens(int n, int n_vocab, int32_t *out);
/* A model file's id in .ts5ref files (engine/src/checks.cpp:39-50): its size and a 64-bit hash of
 * its first MiB (FNV-1a steps from ts5's start value 1469598103934665603). */
int ts5hip_model_file_id(const char *path, uint64_t *size, uint64_t *hash);
/* Where a model's saved reference logits live (engine/src/checks.cpp:56-58): MODEL.ts5ref for an
 * f16 cache, MODEL.q8.ts5ref, MODEL.f32.ts5ref. */
int ts5hip_ref_path(const char *model_path, int kv_type, char *out, int len);
/* load_ref / save_ref (engine/src/checks.cpp:73-104) in the reference's file format: the first n
 * positions' logits [n][n_vocab] of a file of this model (size and hash), cache type and at least
 * n positions; saving keeps a file of the same model and cache type that holds more positions. */
int ts5hip_ref_load(const char *model_path, int n, int n_vocab, int kv_type, float *logits);
int ts5hip_ref_save(const char *model_path, int n, int n_vocab, int kv_type, const float *logits);
/* run_check (engine/src/checks.cpp:108-160) on model m: the n test tokens as n - min(4, n/2)
 * positions in one call with every position's logits, then the rest one token per call; against
 * ref_logits ([n][n_vocab], ts5's CPU backend with the same cache rounding) or, when null, the
 * saved file of model_path. Passes when every logit is finite and max |diff| is under 0.5 % of the
 * largest reference logit (2 % with a q8 cache). */
int ts5hip_check_run(ts5hip_model *m, const char *model_path, int n, const float *ref_logits,
                     ts5hip_check_result *r);

/* ---- the decode driver: Engine (engine/src/engine.h:33-66) over this backend ---- */

typedef struct ts5hip_engine ts5hip_engine;
/* SampleParams (engine/src/engine.h:16-23). draft < 0: 7 drafted tokens per step; 0: none.
 * adapt: the adaptive draft length (TS5_ADAPT, engine/src/engine.cpp:225-228). seed 0 keeps the
 * generator's state (std::mt19937_64, default-seeded when the engine is made). */
typedef struct {
    float temperature, top_p;
    int32_t top_k, max_tokens;
    uint64_t seed;
    int32_t draft, adapt;
} ts5hip_sample_params;
/* Engine(Model, Backend, Tokenizer): generation over model m, which must outlive it. */
int ts5hip_engine_new(ts5hip_model *m, ts5hip_engine **out);
void ts5hip_engine_free(ts5hip_engine *e);
/* Engine::set_drafter (engine/src/engine.cpp:59-68): dm's greedy continuations become the
 * drafts where prompt lookup finds none (null: none). dm is not owned and must outlive e;
 * its token ids must be the target's. */
int ts5hip_engine_set_drafter(ts5hip_engine *e, ts5hip_model *dm);
/* Engine::generate (engine/src/engine.cpp:149-292) with the tokens as ids instead of text:
 * the prompt in 256-token chunks after the prefix already cached, then per step the next token
 * and up to `draft` drafts (prompt lookup, engine.cpp:134-147, else the draft model,
 * engine.cpp:75-129) forwarded as one batch, each draft kept while the sample at its position
 * equals it. eog: n_eog end-of-generation ids. out: the generated ids (at most max_tokens);
 * returns their count, or a negative error. stats (6): prompt tokens, prompt tokens evaluated,
 * generated, drafted, accepted drafts, 1 if an end-of-generation id stopped it. */
int ts5hip_engine_generate(ts5hip_engine *e, const int32_t *prompt, int n_prompt, const ts5hip_sample_params *p,
                           const int32_t *eog, int n_eog, int32_t *out, int32_t *stats);
/* The draft model's state (Engine::drafter_ok_, engine/src/engine.h:70; set false with the
 * "draft model stopped/failed" lines of engine/src/engine.cpp:82-87, :97-101, :117-121):
 * 0 no draft model, 1 drafting, 2 stopped for the rest of the engine's life (a history token past
 * its embedding rows, or one of its forwards failed). Drafts the drafter picks past the target's
 * vocabulary are dropped one at a time and do not stop it. */
int ts5hip_engine_drafter_state(const ts5hip_engine *e);
/* The last generate call's drafts by source (the split behind stats' drafted / accepted, which
 * ts5 prints as one "draft a/b accepted" figure, engine/src/cli.cpp:364-366): out[4] = drafted by
 * prompt lookup, of those accepted, drafted by the draft model, of those accepted. */
int ts5hip_engine_draft_sources(const ts5hip_engine *e, int32_t *out);

#ifdef __cplusplus
}
#endif
#endif /* TS5HIP_H */
