// The model behind the C ABI: tensors by GGUF name, the q8 KV cache, and the
// token forward of ts5's Backend (engine/src/backend.h:16-44) as a sequence
// of HIP kernels captured once into HIP graphs and replayed per token (the
// counterpart of VkBackend::record / record-ahead,
// engine/src/vk_backend.cpp:1049-1199).
//
// One token at position p (state[0] = p, its id at seq[p]):
//   embed -> per layer: act(rmsnorm x) -> QKV matvec -> RoPE + q8 KV append
//   -> split-K flash decode + merge (act) -> O matvec (x +=) -> act(rmsnorm x)
//   -> gate/up + SiLU (act) -> down matvec (x +=)
//   -> act(rmsnorm x) -> head matvec -> logits [-> argmax -> seq[p+1]], p++.
// The token id and position live in device memory, so one graph serves every
// step, and greedy decoding never returns to the host between tokens.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "common_host.h"
#include "kernels.h"
#include "runtime.h"


using namespace ts5hip;

namespace {

struct DevT {
    uint32_t type = 0;   // the HBM layout the kernels read (device_type of gtype)
    uint32_t gtype = 0;  // the GGML type the tensor came in
    int64_t ne0 = 0, ne1 = 0;
    void *d = nullptr;
    bool set = false;
};

struct LayerDev {
    DevT attn_norm, ffn_norm, q_norm, k_norm;
    DevT post_attn_norm, post_ffn_norm;  // Gemma 3: norms of the attention / FFN output
    DevT qkv;                    // [q; k; v] rows of one type
    DevT part[3];                // a q/k/v matrix whose type differs from qkv's
    bool in_qkv[3] = {false, false, false};
    bool qkv_done[3] = {false, false, false};  // every row of the part in qkv has been set
    bool qkv_apart = false;  // q, k and v of different types with a split layout: each in its own buffer
    DevT wo, gate, up, down;
};

enum Graph { G_KV = 0, G_LOGITS = 1, G_GREEDY = 2, N_GRAPHS = 3 };

}  // namespace

struct ts5hip_model {
    ts5hip_ctx *ctx = nullptr;
    ts5hip_hparams hp{};
    int n_ctx = 0, kv_type = KV_Q8, n_split = 1;
    DevT tok_embd, out_norm, output;
    std::vector<float> freqs;
    std::vector<LayerDev> layers;
    float *bias = nullptr;  // [n_layer][(H + 2 HKV) HD], zero where absent
    std::vector<bool> has_bias;
    // KV cache (all layers) and RoPE table. q8: k8 / v8 int8 values with f16
    // scales ks / vs; f16: k8 / v8 hold the halves (2 bytes a value), no scales.
    int8_t *k8 = nullptr, *v8 = nullptr;
    uint16_t *ks = nullptr, *vs = nullptr;
    float *rope_cs = nullptr;
    float *rope_cs_swa = nullptr;  // the sliding layers' (rope_base_swa, no position scaling)
    bool rope_ready = false;
    // Activations and scratch.
    float *x = nullptr, *qkv = nullptr, *att = nullptr, *ffn = nullptr, *logits = nullptr, *part = nullptr;
    float *otmp = nullptr;  // a projection's output before its post-norm (Gemma 3)
    int *counters = nullptr;  // HKV attention merges (CTR_STRIDE apart), then the head argmax's; zero between launches
    void *amax = nullptr;
    int32_t *seq = nullptr;    // [n_ctx + 1] token id at each position
    int32_t *state = nullptr;  // [0] position, [1] last argmax
    // Logits rows of the last forward: on the device, and in pinned host memory
    // (copied there only when a caller reads them on the host).
    float *dev_rows = nullptr, *host_rows = nullptr;
    int rows_cap = 0, rows_valid = 0;
    bool host_fresh = false;
    // GPU picks over those rows: top-k / argmax scratch and results, for up to
    // rows_cap rows of PICK_K candidates (allocated with the rows).
    void *pick_scratch = nullptr;
    float *pick_v = nullptr;
    int32_t *pick_i = nullptr;
    int32_t *pinned_ids = nullptr;  // [n_ctx + 1]
    hipGraphExec_t graph[N_GRAPHS] = {nullptr, nullptr, nullptr};
    bool graphs_stale = true;
    // Verify batches (2..ATTN_MAX_NEW tokens) captured once per token count
    // and logits rows (none, the last, all), replayed like a token's graph.
    // With the per-kernel profile, a graph's own events: [0] before its
    // first kernel, [i] after kernel i (recorded as event nodes of the graph,
    // timed at every replay), and what kernel i was.
    struct GraphProf {
        std::vector<hipEvent_t> ev;
        std::vector<std::string> label;
    };
    GraphProf gprof[N_GRAPHS];
    GraphProf *prof_cap = nullptr;  // the graph being captured
    struct BatchGraph {
        int nc = 0, rows = 0;
        const float *out = nullptr;  // the logits rows it writes (reallocated rows: captured again)
        hipGraphExec_t exec = nullptr;
        GraphProf prof;
    };
    std::vector<BatchGraph> bgraphs;
    bool use_graphs = true;  // TS5HIP_GRAPHS=0: launch each token's kernels directly (profilers)
    // Several tokens per call (prompt chunks, speculative verification): the
    // chunk's activations [CHUNK][...], its quantized activations, the
    // matmul's split-K partials, attention partials and merge counters.
    float *bx = nullptr, *bqkv = nullptr, *bq = nullptr, *batt = nullptr, *bffn = nullptr, *bpart = nullptr;
    float *botmp = nullptr;
    void *bact = nullptr, *bgemm = nullptr;
    int *bcounters = nullptr;
    // Profile (TS5_PROFILE or TS5HIP_PROFILE, engine/src/vk_backend.cpp:347-358):
    // 1 = GPU time of every kernel launch, by kernel and weight role (an event
    // after each launch; in a graph, an event node after each kernel, read
    // after every replay); another nonzero value = GPU time of whole forward
    // calls only.
    int profile = 0;
    double prof_ms = 0;
    int prof_calls = 0, prof_tokens = 0;
    std::vector<hipEvent_t> prof_ev;      // event pool: [0] before the first launch, [i] after launch i
    std::vector<std::string> prof_label;  // what launch i was
    int prof_used = 0;                    // events recorded since the last fold
    std::map<std::string, std::pair<double, int>> prof_kernels;  // label -> (ms, launches)
    std::vector<void *> allocs;

    int qkv_rows() const { return (hp.n_head + 2 * hp.n_head_kv) * hp.head_dim; }
    // A sliding layer (engine/src/model.h:41): the last swa_window keys only.
    bool swa(int l) const {
        return hp.swa_window > 0 && hp.swa_pattern > 0 && l % hp.swa_pattern < hp.swa_pattern - 1;
    }
    int win(int l) const { return swa(l) ? hp.swa_window : 0; }
    const float *rope_of(int l) const { return swa(l) ? rope_cs_swa : rope_cs; }
    // GELU for SiLU in the gate/up's mode (Gemma 3).
    int glu_mode() const { return 2 | (hp.gelu ? GLU_GELU : 0); }
    int64_t kv_head_elems() const { return (int64_t)n_ctx * hp.head_dim; }
    bool kv_f16() const { return kv_type == KV_F16; }
    KvLayer kv_layer(int l) const {
        const int64_t per = (int64_t)hp.n_head_kv * n_ctx * hp.head_dim;
        if (kv_f16()) return KvLayer{k8 + 2 * l * per, nullptr, v8 + 2 * l * per, nullptr};
        const int64_t per_s = per / 32;
        return KvLayer{k8 + l * per, ks + l * per_s, v8 + l * per, vs + l * per_s};
    }
};

namespace {

int alloc(ts5hip_model *m, size_t bytes, void **p) {
    TS5_HIP(m->ctx, hipMalloc(p, bytes ? bytes : 1));
    m->allocs.push_back(*p);
    return TS5HIP_OK;
}

template <typename T>
int alloc_t(ts5hip_model *m, size_t count, T **p) {
    void *v = nullptr;
    if (int rc = alloc(m, count * sizeof(T), &v)) return rc;
    *p = (T *)v;
    return TS5HIP_OK;
}

// ---- the per-kernel profile ----------------------------------------------------
constexpr int PROF_EVENTS = 4096;  // launches timed between two folds

std::string type_tag(uint32_t t) {
    switch (t) {
    case T_F32: return "f32";
    case T_F16: return "f16";
    case T_Q8_0: return "q8_0";
    case T_Q8SM: return "q8sm";
    case T_Q4_K: return "q4_k";
    case T_Q6_K: return "q6_k";
    default: return "t" + std::to_string(t);
    }
}

// Adds the recorded launches' times to prof_kernels. The last event stays as
// the start of the launches that follow.
int prof_fold(ts5hip_model *m) {
    if (m->profile != 1 || m->prof_used < 2) return TS5HIP_OK;
    ts5hip_ctx *ctx = m->ctx;
    const size_t last = (size_t)m->prof_used - 1;
    TS5_HIP(ctx, hipEventSynchronize(m->prof_ev[last]));
    for (size_t i = 1; i <= last; i++) {
        float ms = 0;
        TS5_HIP(ctx, hipEventElapsedTime(&ms, m->prof_ev[i - 1], m->prof_ev[i]));
        auto &e = m->prof_kernels[m->prof_label[i]];
        e.first += ms, e.second++;
    }
    std::swap(m->prof_ev[0], m->prof_ev[last]);
    m->prof_used = 1;
    return TS5HIP_OK;
}

int prof_event(ts5hip_model *m, const std::string &label) {
    ts5hip_ctx *ctx = m->ctx;
    if (m->prof_ev.size() <= (size_t)m->prof_used) {
        hipEvent_t e;
        TS5_HIP(ctx, hipEventCreate(&e));
        m->prof_ev.push_back(e);
        m->prof_label.emplace_back();
    }
    m->prof_label[(size_t)m->prof_used] = label;
    TS5_HIP(ctx, hipEventRecord(m->prof_ev[(size_t)m->prof_used++], ctx->stream));
    return TS5HIP_OK;
}

// The start event of a forward call's launches (none while one is open).
int prof_start(ts5hip_model *m) {
    if (m->profile != 1 || m->prof_used > 0) return TS5HIP_OK;
    return prof_event(m, std::string());
}

// Folds a forward call's launches; the next call starts its own timing.
int prof_close(ts5hip_model *m) {
    if (int rc = prof_fold(m)) return rc;
    m->prof_used = 0;
    return TS5HIP_OK;
}

// An event of the graph being captured (an event node), labelled.
int prof_node(ts5hip_model *m, const std::string &label) {
    ts5hip_ctx *ctx = m->ctx;
    hipEvent_t e;
    TS5_HIP(ctx, hipEventCreate(&e));
    m->prof_cap->ev.push_back(e);
    m->prof_cap->label.push_back(label);
    TS5_HIP(ctx, hipEventRecordWithFlags(e, ctx->stream, hipEventRecordExternal));
    return TS5HIP_OK;
}

void prof_clear(ts5hip_model::GraphProf &gp) {
    for (hipEvent_t e : gp.ev) (void)hipEventDestroy(e);
    gp.ev.clear();
    gp.label.clear();
}

// Starts the events of a graph about to be captured (profile 1).
int prof_capture(ts5hip_model *m, ts5hip_model::GraphProf *gp) {
    if (m->profile != 1) return TS5HIP_OK;
    prof_clear(*gp);
    m->prof_cap = gp;
    return prof_node(m, std::string());
}

// After a replay of a graph captured with events: waits for it and adds its
// kernels' times.
int prof_replayed(ts5hip_model *m, const ts5hip_model::GraphProf &gp) {
    if (m->profile != 1 || gp.ev.size() < 2) return TS5HIP_OK;
    ts5hip_ctx *ctx = m->ctx;
    TS5_HIP(ctx, hipEventSynchronize(gp.ev.back()));
    for (size_t i = 1; i < gp.ev.size(); i++) {
        float ms = 0;
        TS5_HIP(ctx, hipEventElapsedTime(&ms, gp.ev[i - 1], gp.ev[i]));
        auto &e = m->prof_kernels[gp.label[i]];
        e.first += ms, e.second++;
    }
    return TS5HIP_OK;
}

// The event after the launch just enqueued, labelled "kernel role".
int prof_stamp(ts5hip_model *m, const std::string &kernel, const char *role) {
    if (m->profile != 1) return TS5HIP_OK;
    if (m->prof_cap) return prof_node(m, role && *role ? kernel + " " + role : kernel);
    if (m->prof_used == 0)
        if (int rc = prof_start(m)) return rc;  // a launch outside a forward call: timed from here on
    if (int rc = prof_event(m, role && *role ? kernel + " " + role : kernel)) return rc;
    return m->prof_used >= PROF_EVENTS ? prof_fold(m) : TS5HIP_OK;
}

// A vector tensor (norm weight, bias, rope freqs) as floats on the host.
int host_floats(ts5hip_ctx *ctx, uint32_t type, int64_t n, const void *src, std::vector<float> &out) {
    out.resize((size_t)n);
    if (type == T_F32) {
        std::memcpy(out.data(), src, (size_t)n * 4);
    } else if (type == T_F16) {
        const uint16_t *h = (const uint16_t *)src;
        for (int64_t i = 0; i < n; i++) {
            const uint32_t s = (uint32_t)(h[i] >> 15) << 31;
            uint32_t e = (h[i] >> 10) & 31u, f = h[i] & 0x3ffu, bits;
            if (e == 31) bits = s | 0x7f800000u | (f << 13);
            else if (e) bits = s | ((e + 112u) << 23) | (f << 13);
            else if (!f) bits = s;
            else {
                int sh = 0;
                while (!(f & 0x400u)) f <<= 1, sh++;
                bits = s | ((uint32_t)(113 - sh) << 23) | ((f & 0x3ffu) << 13);
            }
            std::memcpy(&out[i], &bits, 4);
        }
    } else {
        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "vector tensor of type %u", type);
    }
    return TS5HIP_OK;
}

// Allocates t (once) for a matrix of this shape and type.
int matrix_slot(ts5hip_model *m, DevT &t, uint32_t type, int64_t ne0, int64_t ne1) {
    if (ts5hip_weight_bytes(type, ne0, ne1) < 0 || !ts5hip_supports_type(type) || ne0 % 32)
        return fail(m->ctx, TS5HIP_ERR_UNSUPPORTED, "matrix of type %u, %lld x %lld", type, (long long)ne1,
                    (long long)ne0);
    if (t.d && (t.gtype != type || t.ne0 != ne0 || t.ne1 != ne1)) return fail(m->ctx, TS5HIP_ERR_ARG, "tensor reshaped");
    if (!t.d) {
        if (int rc = alloc(m, device_bytes(type, ne0, ne1), &t.d)) return rc;
        t.type = device_type(type), t.gtype = type, t.ne0 = ne0, t.ne1 = ne1;
    }
    return TS5HIP_OK;
}

// Source of a tensor's bytes: GGUF on the host, or a synthesis seed; rows
// [row0, row0 + nrows) of the tensor (nrows < 0: all of them), the GGUF bytes
// being those rows' only.
struct Source {
    const void *gguf;
    uint64_t seed;
    int centered;
    int64_t row0 = 0, nrows = -1;
    int64_t rows(int64_t ne1) const { return nrows < 0 ? ne1 : nrows; }
    bool whole(int64_t ne1) const { return row0 == 0 && rows(ne1) == ne1; }
    bool last(int64_t ne1) const { return row0 + rows(ne1) == ne1; }
};

int fill_rows(ts5hip_model *m, const DevT &t, int64_t row0, int64_t nrows, const Source &src) {
    if (src.gguf) return upload_weight(m->ctx, t.gtype, t.ne0, nrows, src.gguf, t.d, row0, t.ne1);
    if (t.type != t.gtype) return fail(m->ctx, TS5HIP_ERR_UNSUPPORTED, "synthetic weights of type %u", t.gtype);
    const SplitDst d = split_dst(t.type, t.ne0, t.ne1, t.d, row0);
    TS5_HIP(m->ctx, launch_synth(t.type, t.ne0, nrows, src.seed, src.centered, d.body, d.scales, m->ctx->stream));
    return TS5HIP_OK;
}

int set_matrix(ts5hip_model *m, DevT &t, uint32_t type, int64_t ne0, int64_t ne1, int64_t want0, int64_t want1,
               const Source &src, const char *name) {
    if (ne0 != want0 || ne1 != want1)
        return fail(m->ctx, TS5HIP_ERR_ARG, "%s is %lld x %lld, expected %lld x %lld", name, (long long)ne0,
                    (long long)ne1, (long long)want0, (long long)want1);
    if (src.row0 < 0 || src.row0 + src.rows(ne1) > ne1)
        return fail(m->ctx, TS5HIP_ERR_ARG, "%s: rows %lld.. past %lld", name, (long long)src.row0, (long long)ne1);
    if (int rc = matrix_slot(m, t, type, ne0, ne1)) return rc;
    if (int rc = fill_rows(m, t, src.row0, src.rows(ne1), src)) return rc;
    if (src.last(ne1)) t.set = true;
    return TS5HIP_OK;
}

// Synthesised vectors: N(1, 0.02) generated on the device.
int set_vector(ts5hip_model *m, DevT &t, uint32_t type, int64_t n, int64_t want, const Source &src,
               const char *name) {
    if (n != want) return fail(m->ctx, TS5HIP_ERR_ARG, "%s has %lld values, expected %lld", name, (long long)n,
                               (long long)want);
    if (!src.whole(1)) return fail(m->ctx, TS5HIP_ERR_ARG, "%s: a vector is set whole", name);
    if (!t.d) {
        if (int rc = alloc(m, (size_t)n * 4, &t.d)) return rc;
        t.type = T_F32, t.ne0 = n, t.ne1 = 1;
    }
    if (src.gguf) {
        std::vector<float> f;
        if (int rc = host_floats(m->ctx, type, n, src.gguf, f)) return rc;
        if (int rc = ts5hip_upload(m->ctx, t.d, f.data(), (size_t)n * 4)) return rc;
    } else {
        TS5_HIP(m->ctx, launch_synth(T_F32, n, 1, src.seed, 0, t.d, nullptr, m->ctx->stream));
    }
    t.set = true;
    return TS5HIP_OK;
}

// q, k and v of different types where the shared buffer has a split layout:
// the parts already in it move to buffers of their own (a split layout's
// matvec finds a tensor's scales right behind its own quants), and the
// layer's q, k and v stay apart from then on.
int unfuse_qkv(ts5hip_model *m, LayerDev &L) {
    const ts5hip_hparams &hp = m->hp;
    const int64_t E = hp.n_embd, rows[3] = {(int64_t)hp.n_head * hp.head_dim, (int64_t)hp.n_head_kv * hp.head_dim,
                                            (int64_t)hp.n_head_kv * hp.head_dim};
    const int64_t row0[3] = {0, rows[0], rows[0] + rows[1]};
    const uint32_t t = L.qkv.type;
    for (int p = 0; p < 3; p++) {
        if (!L.in_qkv[p]) continue;
        DevT &d = L.part[p];
        if (int rc = matrix_slot(m, d, L.qkv.gtype, E, rows[p])) return rc;
        const SplitDst from = split_dst(t, E, m->qkv_rows(), L.qkv.d, row0[p]), to = split_dst(t, E, rows[p], d.d, 0);
        const int64_t nb = E / block_values(t) * rows[p];
        TS5_HIP(m->ctx, hipMemcpyAsync(to.body, from.body, (size_t)nb * (t == T_Q6_K ? Q6K_BODY : Q8_BODY),
                                       hipMemcpyDeviceToDevice, m->ctx->stream));
        TS5_HIP(m->ctx, hipMemcpyAsync(to.scales, from.scales, (size_t)nb * split_scale_bytes(t),
                                       hipMemcpyDeviceToDevice, m->ctx->stream));
        d.set = L.qkv_done[p];
        L.in_qkv[p] = false;
    }
    L.qkv_apart = true;
    return TS5HIP_OK;
}

int set_tensor(ts5hip_model *m, const char *name, uint32_t type, int64_t ne0, int64_t ne1, const Source &src) {
    const ts5hip_hparams &hp = m->hp;
    const int64_t E = hp.n_embd, F = hp.n_ff, HD = hp.head_dim, H = hp.n_head, HKV = hp.n_head_kv;
    m->graphs_stale = true;
    const std::string n(name);
    if (n == "token_embd.weight") {
        if (type != T_F32 && type != T_F16 && !ts5hip_supports_type(type))
            return fail(m->ctx, TS5HIP_ERR_UNSUPPORTED, "token_embd of type %u", type);
        if (ne0 != E || ne1 != hp.n_vocab) return fail(m->ctx, TS5HIP_ERR_ARG, "token_embd shape");
        if (src.row0 < 0 || src.row0 + src.rows(ne1) > ne1) return fail(m->ctx, TS5HIP_ERR_ARG, "token_embd rows");
        if (!m->tok_embd.d) {
            const size_t bytes = (type == T_F32 || type == T_F16) ? (size_t)ne0 * ne1 * (type == T_F32 ? 4 : 2)
                                                                  : device_bytes(type, ne0, ne1);
            if (int rc = alloc(m, bytes, &m->tok_embd.d)) return rc;
            m->tok_embd.type = device_type(type), m->tok_embd.gtype = type, m->tok_embd.ne0 = ne0, m->tok_embd.ne1 = ne1;
        } else if (m->tok_embd.gtype != type) {
            return fail(m->ctx, TS5HIP_ERR_ARG, "tensor reshaped");
        }
        if (type == T_F32 || type == T_F16) {
            if (!src.gguf) return fail(m->ctx, TS5HIP_ERR_UNSUPPORTED, "synthetic float embeddings");
            const size_t vb = type == T_F32 ? 4 : 2;
            if (int rc = ts5hip_upload(m->ctx, (uint8_t *)m->tok_embd.d + (size_t)src.row0 * ne0 * vb, src.gguf,
                                       (size_t)ne0 * src.rows(ne1) * vb))
                return rc;
        } else if (int rc = fill_rows(m, m->tok_embd, src.row0, src.rows(ne1), src)) {
            return rc;
        }
        if (src.last(ne1)) m->tok_embd.set = true;
        return TS5HIP_OK;
    }
    if (n == "output_norm.weight") return set_vector(m, m->out_norm, type, ne0 * ne1, E, src, name);
    if (n == "output.weight") return set_matrix(m, m->output, type, ne0, ne1, E, hp.n_vocab, src, name);
    if (n == "rope_freqs.weight") {
        if (!src.gguf) return fail(m->ctx, TS5HIP_ERR_UNSUPPORTED, "synthetic rope_freqs");
        if (!src.whole(1)) return fail(m->ctx, TS5HIP_ERR_ARG, "%s: a vector is set whole", name);
        if (ne0 * ne1 != hp.rope_dims / 2) return fail(m->ctx, TS5HIP_ERR_ARG, "rope_freqs has %lld values", (long long)(ne0 * ne1));
        m->rope_ready = false;
        return host_floats(m->ctx, type, ne0 * ne1, src.gguf, m->freqs);
    }
    int l = -1, used = 0;
    char rest[96] = {0};
    if (std::sscanf(name, "blk.%d.%95s%n", &l, rest, &used) != 2 || l < 0 || l >= hp.n_layer)
        return fail(m->ctx, TS5HIP_ERR_ARG, "unknown tensor %s", name);
    LayerDev &L = m->layers[l];
    const std::string r(rest);
    if (r == "attn_norm.weight") return set_vector(m, L.attn_norm, type, ne0 * ne1, E, src, name);
    if (r == "ffn_norm.weight") return set_vector(m, L.ffn_norm, type, ne0 * ne1, E, src, name);
    if (r == "attn_q_norm.weight") return set_vector(m, L.q_norm, type, ne0 * ne1, HD, src, name);
    if (r == "attn_k_norm.weight") return set_vector(m, L.k_norm, type, ne0 * ne1, HD, src, name);
    if (r == "post_attention_norm.weight") return set_vector(m, L.post_attn_norm, type, ne0 * ne1, E, src, name);
    if (r == "post_ffw_norm.weight") return set_vector(m, L.post_ffn_norm, type, ne0 * ne1, E, src, name);
    if (r == "attn_output.weight") return set_matrix(m, L.wo, type, ne0, ne1, H * HD, E, src, name);
    if (r == "ffn_gate.weight") return set_matrix(m, L.gate, type, ne0, ne1, E, F, src, name);
    if (r == "ffn_up.weight") return set_matrix(m, L.up, type, ne0, ne1, E, F, src, name);
    if (r == "ffn_down.weight") return set_matrix(m, L.down, type, ne0, ne1, F, E, src, name);
    const char *parts[3] = {"attn_q", "attn_k", "attn_v"};
    const int64_t rows[3] = {H * HD, HKV * HD, HKV * HD}, row0[3] = {0, H * HD, (H + HKV) * HD};
    for (int p = 0; p < 3; p++) {
        if (r == std::string(parts[p]) + ".weight") {
            if (ne0 != E || ne1 != rows[p]) return fail(m->ctx, TS5HIP_ERR_ARG, "%s shape", name);
            if (src.row0 < 0 || src.row0 + src.rows(ne1) > ne1) return fail(m->ctx, TS5HIP_ERR_ARG, "%s rows", name);
            if (L.qkv.d && L.qkv.gtype != type && split_layout(L.qkv.type) && !L.qkv_apart)
                if (int rc = unfuse_qkv(m, L)) return rc;
            if (!L.qkv_apart && (!L.qkv.d || L.qkv.gtype == type)) {
                if (int rc = matrix_slot(m, L.qkv, type, E, m->qkv_rows())) return rc;
                if (int rc = fill_rows(m, L.qkv, row0[p] + src.row0, src.rows(ne1), src)) return rc;
                L.in_qkv[p] = true;
                L.part[p].set = false;
                if (src.last(ne1)) L.qkv_done[p] = true;
            } else {
                if (int rc = set_matrix(m, L.part[p], type, ne0, ne1, E, rows[p], src, name)) return rc;
                L.in_qkv[p] = false;
            }
            return TS5HIP_OK;
        }
        if (r == std::string(parts[p]) + ".bias") {
            if (!src.gguf) return fail(m->ctx, TS5HIP_ERR_UNSUPPORTED, "synthetic bias");
            if (!src.whole(1)) return fail(m->ctx, TS5HIP_ERR_ARG, "%s: a vector is set whole", name);
            if (ne0 * ne1 != rows[p]) return fail(m->ctx, TS5HIP_ERR_ARG, "%s shape", name);
            std::vector<float> f;
            if (int rc = host_floats(m->ctx, type, rows[p], src.gguf, f)) return rc;
            m->has_bias[l] = true;
            return ts5hip_upload(m->ctx, m->bias + (int64_t)l * m->qkv_rows() + row0[p], f.data(), f.size() * 4);
        }
    }
    return fail(m->ctx, TS5HIP_ERR_ARG, "unknown tensor %s", name);
}

int check_complete(ts5hip_model *m) {
    auto need = [&](const DevT &t, const char *what, int l) {
        if (t.set) return TS5HIP_OK;
        return l < 0 ? fail(m->ctx, TS5HIP_ERR_STATE, "tensor %s not set", what)
                     : fail(m->ctx, TS5HIP_ERR_STATE, "tensor blk.%d.%s not set", l, what);
    };
    if (int rc = need(m->tok_embd, "token_embd.weight", -1)) return rc;
    if (int rc = need(m->out_norm, "output_norm.weight", -1)) return rc;
    if (!m->output.set && !ts5hip_supports_type(m->tok_embd.gtype))
        return fail(m->ctx, TS5HIP_ERR_UNSUPPORTED, "tied output head of type %u", m->tok_embd.gtype);
    for (int l = 0; l < m->hp.n_layer; l++) {
        const LayerDev &L = m->layers[l];
        if (int rc = need(L.attn_norm, "attn_norm.weight", l)) return rc;
        if (int rc = need(L.ffn_norm, "ffn_norm.weight", l)) return rc;
        const char *parts[3] = {"attn_q.weight", "attn_k.weight", "attn_v.weight"};
        for (int p = 0; p < 3; p++)
            if (!L.in_qkv[p])
                if (int rc = need(L.part[p], parts[p], l)) return rc;
        if (int rc = need(L.wo, "attn_output.weight", l)) return rc;
        if (int rc = need(L.gate, "ffn_gate.weight", l)) return rc;
        if (int rc = need(L.up, "ffn_up.weight", l)) return rc;
        if (int rc = need(L.down, "ffn_down.weight", l)) return rc;
        if (L.gate.type != L.up.type) return fail(m->ctx, TS5HIP_ERR_UNSUPPORTED, "gate and up of different types");
        if (L.post_attn_norm.set != L.post_ffn_norm.set)  // both or neither (cpu_backend.cpp:103)
            return fail(m->ctx, TS5HIP_ERR_STATE, "blk.%d: post_attention_norm and post_ffw_norm go together", l);
    }
    if (!m->rope_ready) {
        const float *ff = m->freqs.empty() ? nullptr : m->freqs.data();
        std::vector<float> t;
        rope_table_host(m->hp.rope_dims, m->n_ctx, m->hp.rope_base, m->hp.rope_scale, ff, t);
        if (int rc = ts5hip_upload(m->ctx, m->rope_cs, t.data(), t.size() * 4)) return rc;
        if (m->rope_cs_swa) {  // cpu_backend.cpp:208: the sliding layers' base, no scaling
            rope_table_host(m->hp.rope_dims, m->n_ctx, m->hp.rope_base_swa, 1.0f, ff, t);
            if (int rc = ts5hip_upload(m->ctx, m->rope_cs_swa, t.data(), t.size() * 4)) return rc;
        }
        m->rope_ready = true;
    }
    return TS5HIP_OK;
}

const char *const kQkvRole[3] = {"attn_q", "attn_k", "attn_v"};

// The kernels of one token at position state[0] (see the file comment).
// tail: 0 = advance the position, 1 = argmax into seq[p+1] and advance.
int enqueue_token(ts5hip_model *m, bool head, int tail) {
    ts5hip_ctx *ctx = m->ctx;
    const hipStream_t s = ctx->stream;
    const ts5hip_hparams &hp = m->hp;
    const int E = hp.n_embd, H = hp.n_head, HKV = hp.n_head_kv, HD = hp.head_dim, F = hp.n_ff;
    const int QR = m->qkv_rows();
#define TS5_STAMP(kernel, role) \
    if (int rc_ = prof_stamp(m, kernel, role)) return rc_
    TS5_HIP(ctx, launch_embed(m->tok_embd.type, m->tok_embd.d, E, hp.n_vocab, m->seq, m->state, 1, m->x, s,
                              hp.embd_scale));
    TS5_STAMP("embed_" + type_tag(m->tok_embd.type), "token_embd");
    for (int l = 0; l < hp.n_layer; l++) {
        const LayerDev &L = m->layers[l];
        const float *an = (const float *)L.attn_norm.d;
        if (L.in_qkv[0] && L.in_qkv[1] && L.in_qkv[2]) {
            TS5_HIP(ctx, launch_matvec(L.qkv.type, L.qkv.d, E, QR, m->x, an, hp.rms_eps, m->qkv, 0, s));
            TS5_STAMP("matvec_" + type_tag(L.qkv.type), "attn_qkv");
        } else {
            // Rows kept in the fused buffer are a sub-tensor only for layouts
            // without a separate scale array (Q4_K); split layouts go per part.
            const int64_t rows[3] = {(int64_t)H * HD, (int64_t)HKV * HD, (int64_t)HKV * HD};
            int64_t r0 = 0;
            for (int p = 0; p < 3; p++) {
                if (L.in_qkv[p]) {
                    if (split_layout(L.qkv.type))  // unfuse_qkv keeps this from happening
                        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "mixed q/k/v types with a split layout");
                    const SplitDst d = split_dst(L.qkv.type, E, QR, L.qkv.d, r0);
                    TS5_HIP(ctx, launch_matvec(L.qkv.type, d.body, E, rows[p], m->x, an, hp.rms_eps, m->qkv + r0, 0, s));
                    TS5_STAMP("matvec_" + type_tag(L.qkv.type), kQkvRole[p]);
                } else {
                    TS5_HIP(ctx, launch_matvec(L.part[p].type, L.part[p].d, E, rows[p], m->x, an, hp.rms_eps,
                                               m->qkv + r0, 0, s));
                    TS5_STAMP("matvec_" + type_tag(L.part[p].type), kQkvRole[p]);
                }
                r0 += rows[p];
            }
        }
        AttnIO io{};
        io.q = m->qkv, io.q_stride = QR, io.rope = 1, io.append = 1;
        io.bias = m->has_bias[l] ? m->bias + (int64_t)l * QR : nullptr;
        io.q_norm = L.q_norm.set ? (const float *)L.q_norm.d : nullptr;
        io.k_norm = L.k_norm.set ? (const float *)L.k_norm.d : nullptr;
        io.eps = hp.rms_eps, io.rope_cs = m->rope_of(l), io.n_rot = hp.rope_dims, io.neox = hp.rope_neox;
        io.kv = m->kv_layer(l), io.kv_f16 = m->kv_f16(), io.kv_per_batch = 0, io.n_ctx = m->n_ctx;
        io.n_keys = m->state, io.B = 1, io.H = H, io.HKV = HKV, io.HD = HD, io.n_split = m->n_split, io.scale = hp.attn_scale;
        io.part = m->part, io.counters = m->counters, io.out = m->att, io.win = m->win(l);
        TS5_HIP(ctx, launch_attn(io, s));
        TS5_STAMP(m->kv_f16() ? "attention_f16" : "attention_q8", "decode");
        // With Gemma 3's post-norms a projection's output is normalized before
        // the residual add (cpu_backend.cpp:250-252, :263-265).
        const bool post = L.post_attn_norm.set;
        TS5_HIP(ctx, launch_matvec(L.wo.type, L.wo.d, (int64_t)H * HD, E, m->att, nullptr, 0.f, post ? m->otmp : m->x,
                                   post ? 0 : 1, s));
        TS5_STAMP("matvec_" + type_tag(L.wo.type), "attn_output");
        if (post) {
            TS5_HIP(ctx, launch_norm_add(m->otmp, E, (const float *)L.post_attn_norm.d, hp.rms_eps, E, 1, m->x, E, s));
            TS5_STAMP("norm_add", "post_attention_norm");
        }
        TS5_HIP(ctx, launch_matvec_glu(L.gate.type, L.gate.d, L.up.d, E, F, m->x, (const float *)L.ffn_norm.d,
                                       hp.rms_eps, m->ffn, s, hp.gelu));
        TS5_STAMP("matvec_glu_" + type_tag(L.gate.type), "ffn_gate+up");
        TS5_HIP(ctx, launch_matvec(L.down.type, L.down.d, F, E, m->ffn, nullptr, 0.f, post ? m->otmp : m->x,
                                   post ? 0 : 1, s));
        TS5_STAMP("matvec_" + type_tag(L.down.type), "ffn_down");
        if (post) {
            TS5_HIP(ctx, launch_norm_add(m->otmp, E, (const float *)L.post_ffn_norm.d, hp.rms_eps, E, 1, m->x, E, s));
            TS5_STAMP("norm_add", "post_ffw_norm");
        }
    }
    if (head) {
        const DevT &out = m->output.set ? m->output : m->tok_embd;
        const char *orole = m->output.set ? "output" : "token_embd";
        const float *on = (const float *)m->out_norm.d;
        if (tail == 1) {
            TS5_HIP(ctx, launch_matvec_argmax(out.type, out.d, E, hp.n_vocab, m->x, on, hp.rms_eps, m->logits, m->amax,
                                              m->counters + HKV * CTR_STRIDE, m->state + 1, m->seq, m->state, s));
            TS5_STAMP("matvec_argmax_" + type_tag(out.type), orole);
            return TS5HIP_OK;
        }
        TS5_HIP(ctx, launch_matvec(out.type, out.d, E, hp.n_vocab, m->x, on, hp.rms_eps, m->logits, 0, s));
        TS5_STAMP("matvec_" + type_tag(out.type), orole);
    }
    TS5_HIP(ctx, launch_advance(m->state, s));
    TS5_STAMP("advance", "");
    return TS5HIP_OK;
}

void drop_batch_graphs(ts5hip_model *m) {
    for (auto &g : m->bgraphs) {
        if (g.exec) (void)hipGraphExecDestroy(g.exec);
        prof_clear(g.prof);
    }
    m->bgraphs.clear();
}

int build_graphs(ts5hip_model *m) {
    if (!m->graphs_stale) return TS5HIP_OK;
    if (int rc = check_complete(m)) return rc;
    if (!m->bgraphs.empty()) {
        TS5_HIP(m->ctx, hipStreamSynchronize(m->ctx->stream));
        drop_batch_graphs(m);
    }
    if (!m->use_graphs) {
        m->graphs_stale = false;
        return TS5HIP_OK;
    }
    ts5hip_ctx *ctx = m->ctx;
    TS5_HIP(ctx, hipStreamSynchronize(ctx->stream));
    for (int g = 0; g < N_GRAPHS; g++) {
        if (m->graph[g]) {
            (void)hipGraphExecDestroy(m->graph[g]);
            m->graph[g] = nullptr;
        }
        hipGraph_t graph = nullptr;
        TS5_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
        int rc = prof_capture(m, &m->gprof[g]);
        if (!rc) rc = enqueue_token(m, g != G_KV, g == G_GREEDY ? 1 : 0);
        m->prof_cap = nullptr;
        const hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
        if (rc) {
            if (graph) (void)hipGraphDestroy(graph);
            return rc;
        }
        if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamEndCapture");
        const hipError_t ei = hipGraphInstantiate(&m->graph[g], graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (ei != hipSuccess) return hip_fail(ctx, ei, "hipGraphInstantiate");
    }
    m->graphs_stale = false;
    return TS5HIP_OK;
}

// One token's kernels: a replay of the captured graph, or direct launches.
int launch_token(ts5hip_model *m, int g) {
    if (!m->use_graphs) return enqueue_token(m, g != G_KV, g == G_GREEDY ? 1 : 0);
    TS5_HIP(m->ctx, hipGraphLaunch(m->graph[g], m->ctx->stream));
    return prof_replayed(m, m->gprof[g]);
}

// Candidates per row of a GPU pick: top-k with k <= PICK_K - 1, plus one more
// to see whether the k-th value is tied with the next.
constexpr int PICK_K = 64;

void free_rows(ts5hip_model *m) {
    if (m->dev_rows) (void)hipFree(m->dev_rows);
    if (m->host_rows) (void)hipHostFree(m->host_rows);
    if (m->pick_scratch) (void)hipFree(m->pick_scratch);
    if (m->pick_v) (void)hipFree(m->pick_v);
    if (m->pick_i) (void)hipFree(m->pick_i);
    m->dev_rows = nullptr, m->host_rows = nullptr, m->pick_scratch = nullptr, m->pick_v = nullptr;
    m->pick_i = nullptr, m->rows_cap = 0, m->rows_valid = 0, m->host_fresh = false;
}

int ensure_rows(ts5hip_model *m, int rows) {
    if (rows <= m->rows_cap) return TS5HIP_OK;
    ts5hip_ctx *ctx = m->ctx;
    TS5_HIP(ctx, hipStreamSynchronize(ctx->stream));
    free_rows(m);
    const int cap = std::max(rows, 8);
    const size_t bytes = (size_t)cap * m->hp.n_vocab * 4;
    const size_t pick = std::max(topk_scratch_bytes(cap), argmax_scratch_bytes(cap));
    TS5_HIP(ctx, hipMalloc((void **)&m->dev_rows, bytes));
    TS5_HIP(ctx, hipHostMalloc((void **)&m->host_rows, bytes, hipHostMallocDefault));
    TS5_HIP(ctx, hipMalloc(&m->pick_scratch, pick));
    TS5_HIP(ctx, hipMalloc((void **)&m->pick_v, (size_t)cap * PICK_K * 4));
    TS5_HIP(ctx, hipMalloc((void **)&m->pick_i, (size_t)cap * PICK_K * 4));
    m->rows_cap = cap;
    return TS5HIP_OK;
}

// The last forward's logits rows in pinned host memory (copied on first use).
int host_rows_ready(ts5hip_model *m) {
    if (m->host_fresh || !m->rows_valid) return TS5HIP_OK;
    ts5hip_ctx *ctx = m->ctx;
    TS5_HIP(ctx, hipMemcpyAsync(m->host_rows, m->dev_rows, (size_t)m->rows_valid * m->hp.n_vocab * 4,
                                hipMemcpyDeviceToHost, ctx->stream));
    TS5_HIP(ctx, hipStreamSynchronize(ctx->stream));
    m->host_fresh = true;
    return TS5HIP_OK;
}

// Positions pos0.. of n tokens; logits rows (all or the last) left at
// dev_rows / host_rows when want_logits.
// Tokens per batched pass: the reference chunks prompts at 256 tokens
// (engine/src/vk_backend.cpp:272-277), and logits_view holds 256 rows.
constexpr int CHUNK = 256;

int ensure_batch(ts5hip_model *m) {
    if (m->bx) return TS5HIP_OK;
    const ts5hip_hparams &hp = m->hp;
    const int64_t E = hp.n_embd, F = hp.n_ff, AH = (int64_t)hp.n_head * hp.head_dim, QR = m->qkv_rows();
    const int64_t wide = std::max({E, F, AH});
    size_t gemm = 0, part = 0;
    const DevT &out = m->output.set ? m->output : m->tok_embd;
    for (int M = 1; M <= CHUNK; M++) {
        auto g = [&](int64_t rows, int64_t ne0, uint32_t t) {
            const int bv = block_values(t) ? block_values(t) : 32;
            gemm = std::max(gemm, gemm_scratch_bytes(rows, M, (int)(ne0 / bv)));
        };
        for (const LayerDev &L : m->layers) {
            g(QR, E, L.qkv.type), g(E, AH, L.wo.type), g(F, E, L.gate.type), g(E, F, L.down.type);
            for (int p = 0; p < 3; p++)
                if (L.part[p].set) g(QR, E, L.part[p].type);
        }
        g(hp.n_vocab, E, out.type);
        part = std::max(part, attn_partial_bytes(M, attn_splits(M, hp.n_head_kv, m->ctx->n_cu), hp.n_head, hp.n_head_kv, hp.head_dim));
        if (attn_mq_fits(M, hp.n_head, hp.n_head_kv, hp.head_dim, m->kv_f16(), 0))
            part = std::max(part, attn_partial_bytes(M, attn_mq_splits(hp.n_head_kv, m->ctx->n_cu), hp.n_head,
                                                     hp.n_head_kv, hp.head_dim));
    }
    part = std::max(part, attn_prefill_partial_bytes(CHUNK, hp.n_head, hp.head_dim, m->n_ctx));
    int rc = 0;
    if ((rc = alloc_t(m, CHUNK * E, &m->bx)) || (rc = alloc_t(m, CHUNK * QR, &m->bqkv)) ||
        (rc = alloc_t(m, CHUNK * AH, &m->bq)) || (rc = alloc_t(m, CHUNK * AH, &m->batt)) ||
        (rc = alloc_t(m, CHUNK * F, &m->bffn)) || (rc = alloc_t(m, CHUNK * E, &m->botmp)) ||
        (rc = alloc(m, CHUNK * std::max({act_bytes(wide), mact_bytes(wide), hact_bytes(wide)}), &m->bact)) ||
        (rc = alloc(m, std::max<size_t>(gemm, 256), &m->bgemm)) || (rc = alloc(m, part, (void **)&m->bpart)) ||
        (rc = alloc_t(m, (size_t)CHUNK * hp.n_head_kv * CTR_STRIDE, &m->bcounters)))
        return rc;
    TS5_HIP(m->ctx, hipMemsetAsync(m->bcounters, 0, (size_t)CHUNK * hp.n_head_kv * CTR_STRIDE * 4, m->ctx->stream));
    return TS5HIP_OK;
}

// nc tokens (ids at seq[p0..]) at positions p0..p0+nc-1 in one pass per
// layer: every projection a matmul over the chunk, attention a causal batch
// over the cache. Logits (rows: 0, 1 = the last token's, nc = all) go to
// `logits` ([rows][n_vocab]).
int enqueue_batch(ts5hip_model *m, int nc, int p0, int rows, float *logits, bool set_pos = true) {
    ts5hip_ctx *ctx = m->ctx;
    const hipStream_t s = ctx->stream;
    const ts5hip_hparams &hp = m->hp;
    const int E = hp.n_embd, H = hp.n_head, HKV = hp.n_head_kv, HD = hp.head_dim, F = hp.n_ff, AH = H * HD;
    const int QR = m->qkv_rows();
    const float eps = hp.rms_eps;
    auto proj = [&](uint32_t t, const void *w, const void *w2, int64_t ne0, int64_t ne1, const float *x,
                    int64_t xstride, const float *norm, int ntok, int mode, float *y, int64_t ldy,
                    const char *role) -> int {
        if (t == T_F16 || t == T_F32) {  // float rows: the one-token matvec per token
            TS5_HIP(ctx, launch_matvec_tokens(t, w, w2, ne0, ne1, x, xstride, norm, eps, ntok, mode, y, ldy, s));
            TS5_STAMP("matvec_" + type_tag(t) + "_tokens", role);
            return TS5HIP_OK;
        }
        if (gemm_fused_fits(t, ne0, ntok)) {
            TS5_HIP(ctx, launch_gemm_fused(w, w2, ne0, ne1, x, xstride, norm, eps, ntok, mode, y, y, ldy, s));
            TS5_STAMP("matmul_fused_" + type_tag(t), role);
            return TS5HIP_OK;
        }
        TS5_HIP(ctx, launch_gemm_act(t, x, xstride, norm, eps, (int)ne0, ntok, m->bact, s));
        TS5_STAMP("act_quant", role);
        TS5_HIP(ctx, launch_gemm(t, w, w2, ne0, ne1, m->bact, ntok, mode, y, y, ldy, m->bgemm, s));
        TS5_STAMP("matmul_" + type_tag(t), role);
        return TS5HIP_OK;
    };
    if (set_pos) {  // a captured batch reads the position its caller stored
        TS5_HIP(ctx, launch_set_pos(m->state, p0, s));
        TS5_STAMP("set_pos", "");
    }
    TS5_HIP(ctx, launch_embed(m->tok_embd.type, m->tok_embd.d, E, hp.n_vocab, m->seq, m->state, nc, m->bx, s,
                              hp.embd_scale));
    TS5_STAMP("embed_" + type_tag(m->tok_embd.type), "token_embd");
    for (int l = 0; l < hp.n_layer; l++) {
        const LayerDev &L = m->layers[l];
        const float *an = (const float *)L.attn_norm.d;
        if (L.in_qkv[0] && L.in_qkv[1] && L.in_qkv[2]) {
            if (int rc = proj(L.qkv.type, L.qkv.d, nullptr, E, QR, m->bx, E, an, nc, 0, m->bqkv, QR, "attn_qkv")) return rc;
        } else {
            const int64_t prow[3] = {(int64_t)AH, (int64_t)HKV * HD, (int64_t)HKV * HD};
            int64_t r0 = 0;
            for (int p = 0; p < 3; p++) {
                if (L.in_qkv[p]) {
                    if (split_layout(L.qkv.type))  // unfuse_qkv keeps this from happening
                        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "mixed q/k/v types with a split layout");
                    const SplitDst d = split_dst(L.qkv.type, E, QR, L.qkv.d, r0);
                    if (int rc = proj(L.qkv.type, d.body, nullptr, E, prow[p], m->bx, E, an, nc, 0, m->bqkv + r0, QR,
                                      kQkvRole[p]))
                        return rc;
                } else {
                    if (int rc = proj(L.part[p].type, L.part[p].d, nullptr, E, prow[p], m->bx, E, an, nc, 0,
                                      m->bqkv + r0, QR, kQkvRole[p]))
                        return rc;
                }
                r0 += prow[p];
            }
        }
        const float *bias = m->has_bias[l] ? m->bias + (int64_t)l * QR : nullptr;
        const float *qn = L.q_norm.set ? (const float *)L.q_norm.d : nullptr;
        const float *kn = L.k_norm.set ? (const float *)L.k_norm.d : nullptr;
        // Batches of up to ATTN_MAX_NEW tokens (verify steps) leave RoPE and the
        // K/V append to the attention's work items; longer chunks round and
        // append first (k_rope_kv) and read the cache.
        const bool fused = nc <= ATTN_MAX_NEW;
        const int win = m->win(l);  // a sliding layer's window, else 0
        const bool post = L.post_attn_norm.set;
        // Up to 5 tokens with the multi-query attention: it also writes wo's
        // activation records, and wo runs on them (k_gemm_mw).
        const bool mq = !win && attn_mq_fits(nc, H, HKV, HD, m->kv_f16(), 0);
        const bool wo_rec = fused && nc <= 5 && L.wo.type == T_Q4_K && AH % 256 == 0 && mq && !post;
        if (!fused) {
            TS5_HIP(ctx, launch_rope_kv(m->bqkv, QR, bias, qn, kn, eps, m->rope_of(l), hp.rope_dims, hp.rope_neox,
                                        m->state, H, HKV, HD, m->n_ctx, nc, m->bq, m->kv_layer(l), m->kv_f16(), s));
            TS5_STAMP("rope_kv_append", "");
        }
        // Prompt chunks on the matrix cores; a sliding layer's chunk (each
        // query its own window) on the per-query kernel.
        if (nc > 16 && !win && attn_prefill_supported(H, HKV, HD)) {
            TS5_HIP(ctx, launch_attn_prefill(m->bq, AH, m->kv_layer(l), m->kv_f16(), m->n_ctx, H, HKV, HD, p0, nc,
                                             hp.attn_scale, m->bpart, m->batt, s));
            TS5_STAMP("attention_prompt", "");
        } else {
            AttnIO io{};
            if (fused) {
                io.q = m->bqkv, io.q_stride = QR, io.rope = 1, io.append = 1;
                io.bias = bias, io.q_norm = qn, io.k_norm = kn, io.eps = eps, io.rope_cs = m->rope_of(l);
                io.n_rot = hp.rope_dims, io.neox = hp.rope_neox;
            } else {
                io.q = m->bq, io.q_stride = AH, io.rope = 0, io.append = 0;
            }
            io.kv = m->kv_layer(l), io.kv_f16 = m->kv_f16(), io.kv_per_batch = 0, io.n_ctx = m->n_ctx;
            io.n_keys = m->state, io.B = nc, io.H = H, io.HKV = HKV, io.HD = HD;
            io.n_split = mq ? attn_mq_splits(HKV, ctx->n_cu) : attn_splits(nc, HKV, ctx->n_cu);
            io.scale = hp.attn_scale, io.part = m->bpart, io.counters = m->bcounters, io.out = m->batt, io.win = win;
            // A verify batch's attention also writes wo's activation records.
            if (wo_rec) io.act_out = m->bact, io.act_stride = (int64_t)gemm_act_bytes(L.wo.type, AH, nc);
            TS5_HIP(ctx, launch_attn(io, s));
            TS5_STAMP(m->kv_f16() ? "attention_f16" : "attention_q8", "batch");
        }
        if (wo_rec) {
            TS5_HIP(ctx, launch_gemm(L.wo.type, L.wo.d, nullptr, AH, E, m->bact, nc, 1, m->bx, m->bx, E, m->bgemm, s));
            TS5_STAMP("matmul_" + type_tag(L.wo.type), "attn_output");
        } else if (int rc = proj(L.wo.type, L.wo.d, nullptr, AH, E, m->batt, AH, nullptr, nc, post ? 0 : 1,
                                 post ? m->botmp : m->bx, E, "attn_output")) {
            return rc;
        }
        if (post) {  // Gemma 3: x += rmsnorm(wo . att) (cpu_backend.cpp:250-252)
            TS5_HIP(ctx, launch_norm_add(m->botmp, E, (const float *)L.post_attn_norm.d, eps, E, nc, m->bx, E, s));
            TS5_STAMP("norm_add", "post_attention_norm");
        }
        // A verify batch's gate/up also writes the down projection's
        // activation records (no separate quantization launch between them).
        const bool down_rec = L.gate.type == T_Q4_K && L.down.type == T_Q4_K && nc <= 5 && !post &&
                              gemm_fused_qout_fits(E, F, nc) && !gemm_fused_fits(L.down.type, F, nc);
        if (down_rec) {
            TS5_HIP(ctx, launch_gemm_fused(L.gate.d, L.up.d, E, F, m->bx, E, (const float *)L.ffn_norm.d, eps, nc,
                                           m->glu_mode(), m->bffn, m->bffn, F, s, m->bact));
            TS5_STAMP("matmul_fused_" + type_tag(L.gate.type), "ffn_gate+up");
            TS5_HIP(ctx, launch_gemm(L.down.type, L.down.d, nullptr, F, E, m->bact, nc, 1, m->bx, m->bx, E, m->bgemm, s));
            TS5_STAMP("matmul_" + type_tag(L.down.type), "ffn_down");
        } else {
            if (int rc = proj(L.gate.type, L.gate.d, L.up.d, E, F, m->bx, E, (const float *)L.ffn_norm.d, nc,
                              m->glu_mode(), m->bffn, F, "ffn_gate+up"))
                return rc;
            if (int rc = proj(L.down.type, L.down.d, nullptr, F, E, m->bffn, F, nullptr, nc, post ? 0 : 1,
                              post ? m->botmp : m->bx, E, "ffn_down"))
                return rc;
            if (post) {  // cpu_backend.cpp:263-265
                TS5_HIP(ctx, launch_norm_add(m->botmp, E, (const float *)L.post_ffn_norm.d, eps, E, nc, m->bx, E, s));
                TS5_STAMP("norm_add", "post_ffw_norm");
            }
        }
    }
    if (rows) {
        const DevT &out = m->output.set ? m->output : m->tok_embd;
        const float *x = rows == nc ? m->bx : m->bx + (int64_t)(nc - 1) * E;
        if (int rc = proj(out.type, out.d, nullptr, E, hp.n_vocab, x, E, (const float *)m->out_norm.d, rows, 0, logits,
                          hp.n_vocab, m->output.set ? "output" : "token_embd"))
            return rc;
    }
    return TS5HIP_OK;
}
#undef TS5_STAMP

// A verify batch of nc tokens at the position in state[0] (set by the
// caller), logits rows 0, 1 (the last) or nc to dev_rows: its captured graph,
// captured on first use.
int launch_batch_graph(ts5hip_model *m, int nc, int rows) {
    ts5hip_ctx *ctx = m->ctx;
    ts5hip_model::BatchGraph *hit = nullptr;
    for (auto &g : m->bgraphs)
        if (g.nc == nc && g.rows == rows) hit = &g;
    if (hit && rows && hit->out != m->dev_rows) {  // the rows were reallocated since the capture
        TS5_HIP(ctx, hipStreamSynchronize(ctx->stream));
        (void)hipGraphExecDestroy(hit->exec);
        hit->exec = nullptr;
    }
    if (!hit || !hit->exec) {
        if (!hit) {
            m->bgraphs.emplace_back();
            hit = &m->bgraphs.back();
            hit->nc = nc, hit->rows = rows;
        }
        hipGraph_t graph = nullptr;
        TS5_HIP(ctx, hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
        int rc = prof_capture(m, &hit->prof);
        if (!rc) rc = enqueue_batch(m, nc, 0, rows, m->dev_rows, false);
        m->prof_cap = nullptr;
        const hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
        if (rc) {
            if (graph) (void)hipGraphDestroy(graph);
            return rc;
        }
        if (e != hipSuccess) return hip_fail(ctx, e, "hipStreamEndCapture");
        hipGraphExec_t exec = nullptr;
        const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (ei != hipSuccess) return hip_fail(ctx, ei, "hipGraphInstantiate");
        hit->out = m->dev_rows, hit->exec = exec;
    }
    TS5_HIP(ctx, hipGraphLaunch(hit->exec, ctx->stream));
    return prof_replayed(m, hit->prof);
}

int run_tokens(ts5hip_model *m, const int32_t *tokens, int n, int pos0, bool want_logits, bool all) {
    ts5hip_ctx *ctx = m->ctx;
    if (!tokens || n <= 0 || pos0 < 0) return fail(ctx, TS5HIP_ERR_ARG, "bad tokens/n/pos0");
    if ((int64_t)pos0 + n > m->n_ctx) return fail(ctx, TS5HIP_ERR_CONTEXT_FULL, "context full");
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= m->hp.n_vocab)
            return fail(ctx, TS5HIP_ERR_ARG, "token %d out of range", tokens[i]);
    if (int rc = build_graphs(m)) return rc;
    const int rows = want_logits ? (all ? n : 1) : 0;
    if (rows)
        if (int rc = ensure_rows(m, rows)) return rc;
    const hipStream_t s = ctx->stream;
    std::memcpy(m->pinned_ids, tokens, (size_t)n * 4);
    m->pinned_ids[n] = pos0;
    TS5_HIP(ctx, hipMemcpyAsync(m->seq + pos0, m->pinned_ids, (size_t)n * 4, hipMemcpyHostToDevice, s));
    TS5_HIP(ctx, hipMemcpyAsync(m->state, m->pinned_ids + n, 4, hipMemcpyHostToDevice, s));
    if (m->profile) TS5_HIP(ctx, hipEventRecord(ctx->ev0, s));
    if (int rc = prof_start(m)) return rc;
    const size_t row_bytes = (size_t)m->hp.n_vocab * 4;
    if (n == 1) {
        if (int rc = launch_token(m, want_logits ? G_LOGITS : G_KV)) return rc;
        if (want_logits)
            TS5_HIP(ctx, hipMemcpyAsync(m->dev_rows, m->logits, row_bytes, hipMemcpyDeviceToDevice, s));
    } else if (m->use_graphs && n <= ATTN_MAX_NEW) {
        if (int rc = ensure_batch(m)) return rc;
        if (int rc = launch_batch_graph(m, n, !want_logits ? 0 : all ? n : 1)) return rc;
        TS5_HIP(ctx, launch_set_pos(m->state, pos0 + n, s));
    } else {
        if (int rc = ensure_batch(m)) return rc;
        for (int c0 = 0; c0 < n; c0 += CHUNK) {
            const int nc = std::min(CHUNK, n - c0);
            const bool last = c0 + nc == n;
            const int r = !want_logits ? 0 : all ? nc : last ? 1 : 0;
            if (int rc = enqueue_batch(m, nc, pos0 + c0, r, m->dev_rows + (all ? (size_t)c0 * m->hp.n_vocab : 0)))
                return rc;
        }
        TS5_HIP(ctx, launch_set_pos(m->state, pos0 + n, s));
        if (int rc = prof_stamp(m, "set_pos", "")) return rc;
    }
    if (m->profile) TS5_HIP(ctx, hipEventRecord(ctx->ev1, s));
    TS5_HIP(ctx, hipStreamSynchronize(s));
    if (m->profile) {
        float ms = 0;
        TS5_HIP(ctx, hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1));
        m->prof_ms += ms, m->prof_calls++, m->prof_tokens += n;
    }
    if (int rc = prof_close(m)) return rc;
    m->rows_valid = rows;
    m->host_fresh = false;
    return TS5HIP_OK;
}

}  // namespace

namespace ts5hip {
int model_vocab(const ts5hip_model *m) { return m->hp.n_vocab; }
ts5hip_ctx *model_ctx(const ts5hip_model *m) { return m->ctx; }

int model_pick_rows(ts5hip_model *m, int row0, int nrows, float temperature, int top_k, RowPicks &pk) {
    ts5hip_ctx *ctx = m->ctx;
    const int nv = m->hp.n_vocab;
    if (row0 < 0 || nrows < 1 || row0 + nrows > m->rows_valid)
        return fail(ctx, TS5HIP_ERR_STATE, "rows %d..%d of %d logits rows", row0, row0 + nrows, m->rows_valid);
    const float *rows = m->dev_rows + (size_t)row0 * nv;
    pk.row0 = row0, pk.nrows = nrows, pk.k = 0, pk.kk = 0;
    if (temperature <= 0) {
        pk.mode = PICK_GREEDY;
        pk.id.resize((size_t)nrows);
        TS5_HIP(ctx, launch_argmax(rows, nv, nrows, m->pick_scratch, m->pick_i, nullptr, nullptr, ctx->stream));
        TS5_HIP(ctx, hipMemcpyAsync(pk.id.data(), m->pick_i, (size_t)nrows * 4, hipMemcpyDeviceToHost, ctx->stream));
        TS5_HIP(ctx, hipStreamSynchronize(ctx->stream));
        return TS5HIP_OK;
    }
    const int k = top_k > 0 ? std::min(top_k, nv) : nv;
    if (k + 1 <= PICK_K && k < nv && nv <= topk_max_n()) {
        pk.mode = PICK_TOPK, pk.k = k, pk.kk = k + 1;
        pk.v.resize((size_t)nrows * pk.kk);
        pk.id.resize((size_t)nrows * pk.kk);
        TS5_HIP(ctx, launch_topk(rows, nv, pk.kk, nrows, m->pick_scratch, m->pick_v, m->pick_i, ctx->stream));
        TS5_HIP(ctx, hipMemcpyAsync(pk.v.data(), m->pick_v, pk.v.size() * 4, hipMemcpyDeviceToHost, ctx->stream));
        TS5_HIP(ctx, hipMemcpyAsync(pk.id.data(), m->pick_i, pk.id.size() * 4, hipMemcpyDeviceToHost, ctx->stream));
        TS5_HIP(ctx, hipStreamSynchronize(ctx->stream));
        return TS5HIP_OK;
    }
    pk.mode = PICK_HOST;
    return host_rows_ready(m);
}

int32_t model_draw(ts5hip_model *m, ts5hip_sampler *s, const RowPicks &pk, int i, float temperature, float top_p,
                   int top_k) {
    const int nv = m->hp.n_vocab;
    if (i < 0 || i >= pk.nrows) return fail(m->ctx, TS5HIP_ERR_ARG, "pick %d of %d", i, pk.nrows);
    if (pk.mode == PICK_GREEDY) return pk.id[(size_t)i];
    if (pk.mode == PICK_TOPK) {
        // Distinct values through the (k+1)-th: the candidate set and its order
        // are the only ones Engine::sample's heap can produce. A tie or a NaN
        // leaves them to the heap's own order: the whole row, on the host.
        const float *v = pk.v.data() + (size_t)i * pk.kk;
        bool distinct = !std::isnan(v[0]);
        for (int j = 1; j < pk.kk && distinct; j++) distinct = !std::isnan(v[j]) && v[j] != v[j - 1];
        if (distinct) return ts5hip_sampler_draw(s, pk.id.data() + (size_t)i * pk.kk, v, pk.k, temperature, top_p);
    }
    if (int rc = host_rows_ready(m)) return rc;
    return sample_host_row(s, m->host_rows + (size_t)(pk.row0 + i) * nv, nv, temperature, top_p, top_k);
}
}  // namespace ts5hip

extern "C" {

int ts5hip_model_create(ts5hip_ctx *ctx, const ts5hip_hparams *hp, int n_ctx, int kv_type, ts5hip_model **out) {
    if (!ctx || !hp || !out) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    *out = nullptr;
    if (kv_type != KV_Q8 && kv_type != KV_F16)
        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "KV type %d (the GPU cache is q8 or f16)", kv_type);
    // Rows are whole 32-value blocks (Q8_0; Q4_K/Q6_K tensors also check ne0 % 256).
    if (hp->n_embd <= 0 || hp->n_embd % 32 || hp->n_ff <= 0 || hp->n_ff % 32 || hp->n_layer <= 0 ||
        hp->n_vocab <= 0 || n_ctx <= 0 || hp->rope_dims <= 0 || hp->rope_dims > hp->head_dim || hp->rope_dims % 2)
        return fail(ctx, TS5HIP_ERR_ARG, "bad hyperparameters");
    if (!attn_supported(hp->n_head, hp->n_head_kv, hp->head_dim))
        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "attention for %d/%d heads of %d", hp->n_head, hp->n_head_kv,
                    hp->head_dim);
    ts5hip_model *m = new ts5hip_model();
    m->ctx = ctx;
    m->hp = *hp;
    m->n_ctx = n_ctx;
    m->kv_type = kv_type;
    m->layers.resize(hp->n_layer);
    m->has_bias.assign(hp->n_layer, false);
    m->n_split = attn_splits(1, hp->n_head_kv, ctx->n_cu);
    const char *prof = std::getenv("TS5_PROFILE");
    if (!prof || !*prof) prof = std::getenv("TS5HIP_PROFILE");
    m->profile = prof && *prof ? std::atoi(prof) : 0;
    const char *graphs = std::getenv("TS5HIP_GRAPHS");
    // Every kernel timed on its own: launched directly, not replayed as a graph.
    m->use_graphs = !(graphs && std::strcmp(graphs, "0") == 0);
    const int64_t E = hp->n_embd, F = hp->n_ff, HD = hp->head_dim, H = hp->n_head, HKV = hp->n_head_kv;
    const int64_t kv_elems = (int64_t)hp->n_layer * HKV * n_ctx * HD;
    int rc = 0;
    const int64_t kv_value_bytes = kv_type == KV_F16 ? 2 : 1, kv_scales = kv_type == KV_F16 ? 0 : kv_elems / 32;
    if ((rc = alloc_t(m, kv_elems * kv_value_bytes, &m->k8)) || (rc = alloc_t(m, kv_elems * kv_value_bytes, &m->v8)) ||
        (kv_scales && ((rc = alloc_t(m, kv_scales, &m->ks)) || (rc = alloc_t(m, kv_scales, &m->vs)))) ||
        (rc = alloc_t(m, (size_t)n_ctx * hp->rope_dims, &m->rope_cs)) ||
        (hp->swa_window > 0 && (rc = alloc_t(m, (size_t)n_ctx * hp->rope_dims, &m->rope_cs_swa))) ||
        (rc = alloc_t(m, E, &m->otmp)) ||
        (rc = alloc_t(m, (size_t)hp->n_layer * m->qkv_rows(), &m->bias)) || (rc = alloc_t(m, E, &m->x)) ||
        (rc = alloc_t(m, m->qkv_rows(), &m->qkv)) || (rc = alloc_t(m, H * HD, &m->att)) ||
        (rc = alloc_t(m, F, &m->ffn)) || (rc = alloc_t(m, hp->n_vocab, &m->logits)) ||
        (rc = alloc_t(m, attn_partial_bytes(1, 64, H, HKV, HD) / 4, &m->part)) ||
        (rc = alloc_t(m, HKV * CTR_STRIDE + ARGMAX_CTR_INTS, &m->counters)) ||
        (rc = alloc(m, matvec_argmax_scratch_bytes(), &m->amax)) ||
        (rc = alloc_t(m, (size_t)n_ctx + 1, &m->seq)) || (rc = alloc_t(m, 4, &m->state))) {
        ts5hip_model_destroy(m);
        return rc;
    }
    hipError_t e;
    if ((e = hipMemsetAsync(m->bias, 0, (size_t)hp->n_layer * m->qkv_rows() * 4, ctx->stream)) != hipSuccess ||
        (e = hipMemsetAsync(m->seq, 0, ((size_t)n_ctx + 1) * 4, ctx->stream)) != hipSuccess ||
        (e = hipMemsetAsync(m->counters, 0, ((size_t)HKV * CTR_STRIDE + ARGMAX_CTR_INTS) * 4, ctx->stream)) != hipSuccess ||
        (e = hipMemsetAsync(m->k8, 0, kv_elems * kv_value_bytes, ctx->stream)) != hipSuccess ||
        (e = hipMemsetAsync(m->v8, 0, kv_elems * kv_value_bytes, ctx->stream)) != hipSuccess ||
        (kv_scales && (e = hipMemsetAsync(m->ks, 0, kv_scales * 2, ctx->stream)) != hipSuccess) ||
        (kv_scales && (e = hipMemsetAsync(m->vs, 0, kv_scales * 2, ctx->stream)) != hipSuccess) ||
        (e = hipHostMalloc((void **)&m->pinned_ids, ((size_t)n_ctx + 2) * 4, hipHostMallocDefault)) != hipSuccess ||
        (e = hipStreamSynchronize(ctx->stream)) != hipSuccess) {
        hip_fail(ctx, e, "model buffers");
        ts5hip_model_destroy(m);
        return TS5HIP_ERR_HIP;
    }
    *out = m;
    return TS5HIP_OK;
}

void ts5hip_model_destroy(ts5hip_model *m) {
    if (!m) return;
    (void)hipStreamSynchronize(m->ctx->stream);
    for (auto &g : m->graph)
        if (g) (void)hipGraphExecDestroy(g);
    drop_batch_graphs(m);
    for (void *p : m->allocs) (void)hipFree(p);
    free_rows(m);
    if (m->pinned_ids) (void)hipHostFree(m->pinned_ids);
    for (hipEvent_t e : m->prof_ev) (void)hipEventDestroy(e);
    for (auto &gp : m->gprof) prof_clear(gp);
    delete m;
}

int ts5hip_model_set_tensor_rows(ts5hip_model *m, const char *name, uint32_t type, int64_t ne0, int64_t ne1,
                                 int64_t row0, int64_t nrows, const void *gguf) {
    if (!m || !name || !gguf || nrows <= 0) return fail(m ? m->ctx : nullptr, TS5HIP_ERR_ARG, "bad argument");
    Source src{gguf, 0, 0};
    src.row0 = row0, src.nrows = nrows;
    return set_tensor(m, name, type, ne0, ne1, src);
}

int ts5hip_model_set_tensor(ts5hip_model *m, const char *name, uint32_t type, int64_t ne0, int64_t ne1,
                            const void *gguf) {
    if (!m || !name || !gguf) return fail(m ? m->ctx : nullptr, TS5HIP_ERR_ARG, "null argument");
    return set_tensor(m, name, type, ne0, ne1, Source{gguf, 0, 0});
}

int ts5hip_model_synth_tensor(ts5hip_model *m, const char *name, uint32_t type, int64_t ne0, int64_t ne1,
                              uint64_t seed, int centered) {
    if (!m || !name) return fail(m ? m->ctx : nullptr, TS5HIP_ERR_ARG, "null argument");
    // One stream per tensor name: FNV-1a of the name mixed into the seed.
    uint64_t h = 1469598103934665603ull;
    for (const char *c = name; *c; c++) h = (h ^ (uint8_t)*c) * 1099511628211ull;
    return set_tensor(m, name, type, ne0, ne1, Source{nullptr, seed ^ h, centered});
}

int ts5hip_forward(ts5hip_model *m, const int32_t *tokens, int n, int pos0, float *logits, int all_logits) {
    if (!m) return fail(nullptr, TS5HIP_ERR_ARG, "null model");
    if (int rc = run_tokens(m, tokens, n, pos0, logits != nullptr, all_logits != 0)) return rc;
    if (logits) {
        if (int rc = host_rows_ready(m)) return rc;
        std::memcpy(logits, m->host_rows, (size_t)m->rows_valid * m->hp.n_vocab * 4);
    }
    return TS5HIP_OK;
}

int ts5hip_forward_in_place(ts5hip_model *m, const int32_t *tokens, int n, int pos0, int all_logits) {
    if (!m) return fail(nullptr, TS5HIP_ERR_ARG, "null model");
    return run_tokens(m, tokens, n, pos0, true, all_logits != 0);
}

const float *ts5hip_logits_view(const ts5hip_model *m) {
    if (!m || !m->rows_valid) return nullptr;
    // The rows are copied to the host here, on first use after a forward: a
    // caller that samples on the GPU (ts5hip_logits_topk) never pays for it.
    if (host_rows_ready(const_cast<ts5hip_model *>(m)) != TS5HIP_OK) return nullptr;
    return m->host_rows;
}
int ts5hip_n_ctx(const ts5hip_model *m) { return m ? m->n_ctx : 0; }
int ts5hip_kv_type(const ts5hip_model *m) { return m ? m->kv_type : -1; }

int ts5hip_token_path(ts5hip_model *m) {
    if (!m) return fail(nullptr, TS5HIP_ERR_ARG, "null model");
    if (int rc = build_graphs(m)) return rc;
    return m->use_graphs ? 1 : 0;
}

int32_t ts5hip_model_sample(ts5hip_model *m, ts5hip_sampler *s, int row, float temperature, float top_p, int top_k) {
    if (!m || !s) return fail(m ? m->ctx : nullptr, TS5HIP_ERR_ARG, "null argument");
    if (row < 0 || row >= m->rows_valid) return fail(m->ctx, TS5HIP_ERR_ARG, "row %d of %d", row, m->rows_valid);
    RowPicks pk;
    if (int rc = model_pick_rows(m, row, 1, temperature, top_k, pk)) return rc;
    return model_draw(m, s, pk, 0, temperature, top_p, top_k);
}

int ts5hip_logits_topk(ts5hip_model *m, int row0, int nrows, int k, float *vals, int32_t *ids) {
    if (!m || !vals || !ids) return fail(m ? m->ctx : nullptr, TS5HIP_ERR_ARG, "null argument");
    if (row0 < 0 || nrows < 1 || row0 + nrows > m->rows_valid)
        return fail(m->ctx, TS5HIP_ERR_ARG, "rows %d..%d of %d", row0, row0 + nrows, m->rows_valid);
    if (k < 1 || k > PICK_K || k > m->hp.n_vocab || m->hp.n_vocab > topk_max_n())
        return fail(m->ctx, TS5HIP_ERR_UNSUPPORTED, "top-%d of %d logits", k, m->hp.n_vocab);
    ts5hip_ctx *ctx = m->ctx;
    TS5_HIP(ctx, launch_topk(m->dev_rows + (size_t)row0 * m->hp.n_vocab, m->hp.n_vocab, k, nrows, m->pick_scratch,
                             m->pick_v, m->pick_i, ctx->stream));
    TS5_HIP(ctx, hipMemcpyAsync(vals, m->pick_v, (size_t)nrows * k * 4, hipMemcpyDeviceToHost, ctx->stream));
    TS5_HIP(ctx, hipMemcpyAsync(ids, m->pick_i, (size_t)nrows * k * 4, hipMemcpyDeviceToHost, ctx->stream));
    TS5_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return TS5HIP_OK;
}

int ts5hip_generate_greedy(ts5hip_model *m, int32_t token, int pos, int n_steps, int32_t *ids_out) {
    if (!m) return fail(nullptr, TS5HIP_ERR_ARG, "null model");
    ts5hip_ctx *ctx = m->ctx;
    if (n_steps <= 0 || pos < 0 || token < 0 || token >= m->hp.n_vocab) return fail(ctx, TS5HIP_ERR_ARG, "bad arguments");
    if ((int64_t)pos + n_steps > m->n_ctx) return fail(ctx, TS5HIP_ERR_CONTEXT_FULL, "context full");
    if (int rc = build_graphs(m)) return rc;
    const hipStream_t s = ctx->stream;
    m->pinned_ids[0] = token;
    m->pinned_ids[1] = pos;
    TS5_HIP(ctx, hipMemcpyAsync(m->seq + pos, m->pinned_ids, 4, hipMemcpyHostToDevice, s));
    TS5_HIP(ctx, hipMemcpyAsync(m->state, m->pinned_ids + 1, 4, hipMemcpyHostToDevice, s));
    if (m->profile) TS5_HIP(ctx, hipEventRecord(ctx->ev0, s));
    if (int rc = prof_start(m)) return rc;
    for (int i = 0; i < n_steps; i++)
        if (int rc = launch_token(m, G_GREEDY)) return rc;
    if (m->profile) TS5_HIP(ctx, hipEventRecord(ctx->ev1, s));
    TS5_HIP(ctx, hipMemcpyAsync(m->pinned_ids, m->seq + pos + 1, (size_t)n_steps * 4, hipMemcpyDeviceToHost, s));
    TS5_HIP(ctx, hipStreamSynchronize(s));
    if (m->profile) {
        float ms = 0;
        TS5_HIP(ctx, hipEventElapsedTime(&ms, ctx->ev0, ctx->ev1));
        m->prof_ms += ms, m->prof_calls++, m->prof_tokens += n_steps;
    }
    if (int rc = prof_close(m)) return rc;
    if (ids_out) std::memcpy(ids_out, m->pinned_ids, (size_t)n_steps * 4);
    m->rows_valid = 0;
    return TS5HIP_OK;
}

int ts5hip_kv_read(ts5hip_model *m, int layer, int which, int pos0, int n, float *out) {
    if (!m || !out) return fail(m ? m->ctx : nullptr, TS5HIP_ERR_ARG, "null argument");
    ts5hip_ctx *ctx = m->ctx;
    if (layer < 0 || layer >= m->hp.n_layer || pos0 < 0 || n <= 0 || pos0 + n > m->n_ctx)
        return fail(ctx, TS5HIP_ERR_ARG, "bad layer/range");
    const int64_t w = (int64_t)m->hp.n_head_kv * m->hp.head_dim;
    float *d = nullptr;
    TS5_HIP(ctx, hipMalloc((void **)&d, (size_t)n * w * 4));
    hipError_t e = launch_kv_read(m->kv_layer(layer), which, m->hp.n_head_kv, m->hp.head_dim, m->n_ctx, pos0, n,
                                  m->kv_f16(), d,
                                  ctx->stream);
    int rc = e == hipSuccess ? ts5hip_download(ctx, out, d, (size_t)n * w * 4) : hip_fail(ctx, e, "kv_read");
    (void)hipFree(d);
    return rc;
}

int ts5hip_kv_write(ts5hip_model *m, int layer, int which, int pos0, int n, const float *in) {
    if (!m || !in) return fail(m ? m->ctx : nullptr, TS5HIP_ERR_ARG, "null argument");
    ts5hip_ctx *ctx = m->ctx;
    if (layer < 0 || layer >= m->hp.n_layer || (which != 0 && which != 1) || pos0 < 0 || n <= 0 || pos0 + n > m->n_ctx)
        return fail(ctx, TS5HIP_ERR_ARG, "bad layer/range");
    if (m->hp.head_dim > 128 || m->hp.head_dim % 32) return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "head_dim %d", m->hp.head_dim);
    const size_t bytes = (size_t)n * m->hp.n_head_kv * m->hp.head_dim * 4;
    float *d = nullptr;
    TS5_HIP(ctx, hipMalloc((void **)&d, bytes));
    hipError_t e = hipMemcpyAsync(d, in, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
        e = launch_kv_write(m->kv_layer(layer), which, m->hp.n_head_kv, m->hp.head_dim, m->n_ctx, pos0, n, m->kv_f16(),
                            d, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    (void)hipFree(d);
    if (e != hipSuccess) return hip_fail(ctx, e, "kv_write");
    return TS5HIP_OK;
}

int ts5hip_take_profile(ts5hip_model *m, char *buf, int len) {
    if (!m || !buf || len <= 0) return fail(m ? m->ctx : nullptr, TS5HIP_ERR_ARG, "bad argument");
    std::string s;
    char line[320];
    if (m->profile && m->prof_calls) {
        std::snprintf(line, sizeof line, "hip: %d forward calls, %d tokens, %.3f ms GPU (%.3f ms/token)\n",
                      m->prof_calls, m->prof_tokens, m->prof_ms, m->prof_ms / std::max(1, m->prof_tokens));
        s = line;
    }
    // Kernels by GPU time, most first: kernel and weight role, ms, share, launches.
    std::vector<std::pair<std::string, std::pair<double, int>>> k(m->prof_kernels.begin(), m->prof_kernels.end());
    std::stable_sort(k.begin(), k.end(), [](const auto &a, const auto &b) { return a.second.first > b.second.first; });
    double total = 0;
    for (const auto &e : k) total += e.second.first;
    if (!k.empty()) {
        std::snprintf(line, sizeof line, "GPU time %.1f ms:\n", total);
        s += line;
    }
    for (const auto &e : k) {
        std::snprintf(line, sizeof line, "  %-32s %9.3f ms %5.1f%% %7d calls\n", e.first.c_str(), e.second.first,
                      total > 0 ? 100.0 * e.second.first / total : 0.0, e.second.second);
        s += line;
    }
    // A buffer too small keeps the profile for a call with a larger one.
    if ((int)s.size() >= len) return fail(m->ctx, TS5HIP_ERR_ARG, "a profile of %zu bytes in a buffer of %d", s.size() + 1, len);
    std::memcpy(buf, s.c_str(), s.size() + 1);
    m->prof_ms = 0, m->prof_calls = 0, m->prof_tokens = 0;
    m->prof_kernels.clear();
    return TS5HIP_OK;
}

}  // extern "C"
