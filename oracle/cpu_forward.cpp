// TEST INFRASTRUCTURE ONLY: part of the CPU oracle (see ts5_oracle.h).
//
// The fp32 CPU forward pass, restated from engine/src/cpu_backend.cpp:
// matmul :18-37, rmsnorm :48-53, rope :57-68, round_kv :78-90,
// CpuBackend::forward :120-146, layer :188-266 (llama / mistral / qwen2 /
// qwen3 / gemma3 layers: optional q/k/v bias and per-head q/k norm; Gemma 3's
// embedding scale, sliding windows with their own RoPE base, GELU and the
// norms after attention and the FFN), gelu :71-73.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "ts5_oracle.h"

namespace {

unsigned thread_count(int threads) {
    if (threads > 0) return (unsigned)threads;
    return std::max(1u, std::thread::hardware_concurrency());
}

// Dequantized copy of a small tensor (norm weights, biases, rope freqs).
std::vector<float> as_floats(const ts5o_tensor &t) {
    std::vector<float> v;
    if (!t.data) return v;
    v.resize((size_t)(t.ne0 * t.ne1));
    ts5o_dequantize_row(t.type, t.data, v.data(), (int64_t)v.size());
    return v;
}

int64_t row_bytes_of(const ts5o_tensor &t) {
    return t.ne0 / ts5o_block_values(t.type) * ts5o_block_bytes(t.type);
}

}  // namespace

extern "C" {

int ts5o_matmul(uint32_t type, const void *W, int64_t rb, int64_t n_in, int64_t n_out, const float *X, int n,
                float *Y, int64_t ystride, int threads) {
    if (ts5o_block_values(type) == 0) return -1;
    const unsigned nt = thread_count(threads);
    const uint8_t *base = (const uint8_t *)W;
    auto work = [&](unsigned t) {
        std::vector<float> w((size_t)n_in);
        for (int64_t r = t; r < n_out; r += nt) {
            ts5o_dequantize_row(type, base + r * rb, w.data(), n_in);
            // Four tokens' sums side by side: each is still one chain of fp64
            // adds in index order (the products are exact), so every result is
            // the reference's bit for bit; the chains only overlap in time.
            int j = 0;
            for (; j + 4 <= n; j += 4) {
                const float *x0 = X + (size_t)j * n_in, *x1 = x0 + n_in, *x2 = x1 + n_in, *x3 = x2 + n_in;
                double a0 = 0, a1 = 0, a2 = 0, a3 = 0;
                for (int64_t i = 0; i < n_in; i++) {
                    const double wi = w[i];
                    a0 += wi * x0[i];
                    a1 += wi * x1[i];
                    a2 += wi * x2[i];
                    a3 += wi * x3[i];
                }
                Y[(size_t)j * ystride + r] = (float)a0;
                Y[(size_t)(j + 1) * ystride + r] = (float)a1;
                Y[(size_t)(j + 2) * ystride + r] = (float)a2;
                Y[(size_t)(j + 3) * ystride + r] = (float)a3;
            }
            for (; j < n; j++) {
                const float *x = X + (size_t)j * n_in;
                double acc = 0;
                for (int64_t i = 0; i < n_in; i++) acc += (double)w[i] * x[i];
                Y[(size_t)j * ystride + r] = (float)acc;
            }
        }
    };
    std::vector<std::thread> pool;
    for (unsigned t = 1; t < nt; t++) pool.emplace_back(work, t);
    work(0);
    for (auto &th : pool) th.join();
    return 0;
}

void ts5o_rmsnorm(float *x, const float *w, int n, float eps) {
    double ss = 0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float inv = 1.0f / std::sqrt((float)(ss / n) + eps);
    for (int i = 0; i < n; i++) x[i] = x[i] * inv * w[i];
}

void ts5o_rope_cs(int n_rot, int pos, float base, const float *freqs, float scale, float *c, float *s) {
    for (int i = 0; i < n_rot / 2; i++) {
        float theta = pos * scale * std::pow(base, -2.0f * i / n_rot);
        if (freqs) theta /= freqs[i];
        c[i] = std::cos(theta);
        s[i] = std::sin(theta);
    }
}

void ts5o_rope(float *v, int n_rot, int pos, float base, int neox, const float *freqs, float scale) {
    for (int i = 0; i < n_rot / 2; i++) {
        float theta = pos * scale * std::pow(base, -2.0f * i / n_rot);
        if (freqs) theta /= freqs[i];
        const float c = std::cos(theta), s = std::sin(theta);
        const int a = neox ? i : 2 * i, b = neox ? i + n_rot / 2 : 2 * i + 1;
        const float x0 = v[a], x1 = v[b];
        v[a] = x0 * c - x1 * s;
        v[b] = x0 * s + x1 * c;
    }
}

void ts5o_round_kv(int kv, float *v, int n) {
    if (kv == TS5O_KV_F16) {
        for (int i = 0; i < n; i++) v[i] = ts5o_fp16_to_fp32(ts5o_fp32_to_fp16(v[i]));
        return;
    }
    if (kv != TS5O_KV_Q8) return;
    for (int b = 0; b + 32 <= n; b += 32) {
        float amax = 0;
        for (int i = 0; i < 32; i++) amax = std::max(amax, std::fabs(v[b + i]));
        const float sc = ts5o_fp16_to_fp32(ts5o_fp32_to_fp16(amax / 127.0f));
        for (int i = 0; i < 32; i++) {
            float q = 0.0f;
            if (sc > 0) q = std::min(127.0f, std::max(-127.0f, std::nearbyint(v[b + i] / sc))) * sc;
            v[b + i] = q;
        }
    }
}

void ts5o_attention(const float *q, const float *kc, const float *vc, int H, int HKV, int HD, int lo, int pos,
                    float scale, float *out) {
    const int KV = HKV * HD;
    std::vector<float> w((size_t)pos + 1);
    for (int h = 0; h < H; h++) {
        const int kh = h / (H / HKV);
        const float *qh = q + (size_t)h * HD;
        float mx = -INFINITY;
        for (int p = lo; p <= pos; p++) {
            double dot = 0;
            const float *k = kc + (size_t)p * KV + (size_t)kh * HD;
            for (int d = 0; d < HD; d++) dot += (double)qh[d] * k[d];
            w[p] = (float)dot * scale;
            mx = std::max(mx, w[p]);
        }
        double sum = 0;
        for (int p = lo; p <= pos; p++) {
            w[p] = std::exp(w[p] - mx);
            sum += w[p];
        }
        for (int d = 0; d < HD; d++) {
            double acc = 0;
            for (int p = lo; p <= pos; p++) acc += w[p] * vc[(size_t)p * KV + (size_t)kh * HD + d];
            out[(size_t)h * HD + d] = (float)(acc / sum);
        }
    }
}

void ts5o_swiglu(float *g, const float *u, int64_t n) {
    for (int64_t i = 0; i < n; i++) g[i] = g[i] / (1.0f + std::exp(-g[i])) * u[i];
}

void ts5o_geglu(float *g, const float *u, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        const float x = g[i];
        g[i] = 0.5f * x * (1.0f + std::tanh(0.7978845608f * (x + 0.044715f * x * x * x))) * u[i];
    }
}

}  // extern "C"

struct ts5o_model {
    ts5o_hparams hp;
    ts5o_tensor tok_embd, output;
    std::vector<ts5o_layer> layers;
    struct Small { std::vector<float> attn, ffn, q, k, bq, bk, bv, post_attn, post_ffn; };
    std::vector<Small> small;
    std::vector<float> out_norm, freqs;
    int n_ctx, kv, threads;
    std::vector<float> kc, vc;  // [layer][n_ctx][n_head_kv*head_dim]

    void matmul(const ts5o_tensor &w, const float *X, int n, float *Y) const {
        ts5o_matmul(w.type, w.data, row_bytes_of(w), w.ne0, w.ne1, X, n, Y, w.ne1, threads);
    }

    void layer(int l, float *x, int n, int pos0) {
        const int E = hp.n_embd, HD = hp.head_dim, H = hp.n_head, HKV = hp.n_head_kv, KV = HKV * HD, F = hp.n_ff;
        const ts5o_layer &L = layers[l];
        const Small &S = small[l];
        std::vector<float> h(x, x + (size_t)n * E), q((size_t)n * H * HD), k((size_t)n * KV), v((size_t)n * KV);
        for (int t = 0; t < n; t++) ts5o_rmsnorm(&h[(size_t)t * E], S.attn.data(), E, hp.rms_eps);
        matmul(L.wq, h.data(), n, q.data());
        matmul(L.wk, h.data(), n, k.data());
        matmul(L.wv, h.data(), n, v.data());
        float *kl = &kc[(size_t)l * n_ctx * KV], *vl = &vc[(size_t)l * n_ctx * KV];
        const float *ff = freqs.empty() ? nullptr : freqs.data();
        // A sliding layer (model.h:41): its own RoPE base, no position scaling,
        // and only the last swa_window keys.
        const bool swa = hp.swa_window > 0 && hp.swa_pattern > 0 && l % hp.swa_pattern < hp.swa_pattern - 1;
        const float base = swa ? hp.rope_base_swa : hp.rope_base, rs = swa ? 1.f : hp.rope_scale;
        for (int t = 0; t < n; t++) {
            float *qt = &q[(size_t)t * H * HD], *kt = &k[(size_t)t * KV], *vt = &v[(size_t)t * KV];
            const int pos = pos0 + t;
            if (!S.bq.empty()) {
                for (int i = 0; i < H * HD; i++) qt[i] += S.bq[i];
                for (int i = 0; i < KV; i++) kt[i] += S.bk[i], vt[i] += S.bv[i];
            }
            for (int hh = 0; hh < H; hh++) {
                if (!S.q.empty()) ts5o_rmsnorm(&qt[hh * HD], S.q.data(), HD, hp.rms_eps);
                ts5o_rope(&qt[hh * HD], hp.rope_dims, pos, base, hp.rope_neox, ff, rs);
            }
            for (int hh = 0; hh < HKV; hh++) {
                if (!S.k.empty()) ts5o_rmsnorm(&kt[hh * HD], S.k.data(), HD, hp.rms_eps);
                ts5o_rope(&kt[hh * HD], hp.rope_dims, pos, base, hp.rope_neox, ff, rs);
            }
            ts5o_round_kv(kv, kt, KV);
            ts5o_round_kv(kv, vt, KV);
            std::memcpy(kl + (size_t)pos * KV, kt, (size_t)KV * 4);
            std::memcpy(vl + (size_t)pos * KV, vt, (size_t)KV * 4);
        }
        std::vector<float> att((size_t)n * H * HD), o((size_t)n * E);
        for (int t = 0; t < n; t++) {
            const int pos = pos0 + t, lo = swa ? std::max(0, pos - hp.swa_window + 1) : 0;
            ts5o_attention(&q[(size_t)t * H * HD], kl, vl, H, HKV, HD, lo, pos, hp.attn_scale,
                           &att[(size_t)t * H * HD]);
        }
        matmul(L.wo, att.data(), n, o.data());
        if (!S.post_attn.empty())
            for (int t = 0; t < n; t++) ts5o_rmsnorm(&o[(size_t)t * E], S.post_attn.data(), E, hp.rms_eps);
        for (size_t i = 0; i < (size_t)n * E; i++) x[i] += o[i];
        h.assign(x, x + (size_t)n * E);
        for (int t = 0; t < n; t++) ts5o_rmsnorm(&h[(size_t)t * E], S.ffn.data(), E, hp.rms_eps);
        std::vector<float> g((size_t)n * F), u((size_t)n * F);
        matmul(L.w_gate, h.data(), n, g.data());
        matmul(L.w_up, h.data(), n, u.data());
        if (hp.gelu)
            ts5o_geglu(g.data(), u.data(), (int64_t)n * F);
        else
            ts5o_swiglu(g.data(), u.data(), (int64_t)n * F);
        matmul(L.w_down, g.data(), n, o.data());
        if (!S.post_ffn.empty())
            for (int t = 0; t < n; t++) ts5o_rmsnorm(&o[(size_t)t * E], S.post_ffn.data(), E, hp.rms_eps);
        for (size_t i = 0; i < (size_t)n * E; i++) x[i] += o[i];
    }
};

extern "C" {

ts5o_model *ts5o_model_new(const ts5o_hparams *hp, const ts5o_tensor *tok_embd, const ts5o_tensor *out_norm,
                           const ts5o_tensor *output, const ts5o_tensor *rope_freqs, const ts5o_layer *layers,
                           int n_ctx, int kv_type, int threads) {
    ts5o_model *m = new ts5o_model();
    m->hp = *hp;
    m->tok_embd = *tok_embd;
    m->output = output && output->data ? *output : *tok_embd;  // tied embeddings
    m->layers.assign(layers, layers + hp->n_layer);
    for (const ts5o_layer &L : m->layers) {
        ts5o_model::Small s;
        s.attn = as_floats(L.attn_norm);
        s.ffn = as_floats(L.ffn_norm);
        s.q = as_floats(L.q_norm);
        s.k = as_floats(L.k_norm);
        s.bq = as_floats(L.bq);
        s.bk = as_floats(L.bk);
        s.bv = as_floats(L.bv);
        s.post_attn = as_floats(L.post_attn_norm);
        s.post_ffn = as_floats(L.post_ffn_norm);
        m->small.push_back(std::move(s));
    }
    m->out_norm = as_floats(*out_norm);
    if (rope_freqs) m->freqs = as_floats(*rope_freqs);
    m->n_ctx = n_ctx;
    m->kv = kv_type;
    m->threads = threads;
    const size_t kvn = (size_t)hp->n_layer * n_ctx * hp->n_head_kv * hp->head_dim;
    m->kc.assign(kvn, 0.f);
    m->vc.assign(kvn, 0.f);
    return m;
}

void ts5o_model_free(ts5o_model *m) { delete m; }

float *ts5o_kv(ts5o_model *m, int which, int layer) {
    const size_t per = (size_t)m->n_ctx * m->hp.n_head_kv * m->hp.head_dim;
    return (which ? m->vc.data() : m->kc.data()) + per * layer;
}

int ts5o_forward(ts5o_model *m, const int32_t *tokens, int n, int pos0, float *logits, int all) {
    if (pos0 + n > m->n_ctx) return -1;
    const int E = m->hp.n_embd;
    std::vector<float> x((size_t)n * E);
    const int64_t rb = row_bytes_of(m->tok_embd);
    for (int t = 0; t < n; t++) {
        ts5o_dequantize_row(m->tok_embd.type, (const uint8_t *)m->tok_embd.data + (int64_t)tokens[t] * rb,
                            x.data() + (size_t)t * E, E);
        if (m->hp.embd_scale > 0)
            for (int i = 0; i < E; i++) x[(size_t)t * E + i] *= m->hp.embd_scale;
    }
    for (int l = 0; l < m->hp.n_layer; l++) m->layer(l, x.data(), n, pos0);
    if (!logits) return 0;
    const int nout = all ? n : 1;
    float *xo = x.data() + (size_t)(n - nout) * E;
    for (int t = 0; t < nout; t++) ts5o_rmsnorm(xo + (size_t)t * E, m->out_norm.data(), E, m->hp.rms_eps);
    m->matmul(m->output, xo, nout, logits);
    return 0;
}

}  // extern "C"
