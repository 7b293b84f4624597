// TEST INFRASTRUCTURE ONLY.
//
// A small C-ABI over ts5's own CPU code, compiled by oracle/Makefile from the
// reference sources where they lie (engine/src/{gguf,quants,model,
// cpu_backend,engine,tokenizer,log,checks}.cpp) into oracle/_ref/libts5ref.so. It is
// used only to write and check golden vectors; nothing of the reference is
// copied into this repository.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "backend.h"
#include "checks.h"
#include "engine.h"
#include "model.h"
#include "quants.h"
#include "tokenizer.h"

using namespace ts5;

namespace {

std::string g_err;

KvType kv_of(int k) { return k == 2 ? KvType::Q8 : k == 1 ? KvType::F16 : KvType::F32; }

struct RefCpu {
    Model model;
    std::unique_ptr<Backend> backend;
};

// A backend that hands out prepared logits, one row per position forwarded,
// so Engine::generate's sampler can be driven on chosen inputs.
class TableBackend : public Backend {
public:
    TableBackend(const float *rows, int n_rows, int n_vocab, int n_ctx)
        : rows_(rows), n_rows_(n_rows), nv_(n_vocab), n_ctx_(n_ctx) {}
    const char *name() const override { return "table"; }
    int n_ctx() const override { return n_ctx_; }
    bool forward(const int32_t *, int n, int, float *logits, bool all, std::string &err) override {
        const int rows = all ? n : 1;
        if (next_ + rows > n_rows_) { err = "table exhausted"; return false; }
        if (logits) std::memcpy(logits, rows_ + (size_t)next_ * nv_, (size_t)rows * nv_ * 4);
        next_ += rows;
        return true;
    }

private:
    const float *rows_;
    int n_rows_, nv_, n_ctx_, next_ = 0;
};

// The CPU backend with the KV rounding of `kv`, reporting that cache type
// (CpuBackend itself reports F32), so run_check treats it as a GPU backend
// with such a cache.
class KvTagged : public Backend {
public:
    KvTagged(Backend *inner, KvType kv) : inner_(inner), kv_(kv) {}
    const char *name() const override { return "cpu"; }
    int n_ctx() const override { return inner_->n_ctx(); }
    KvType kv_type() const override { return kv_; }
    bool forward(const int32_t *t, int n, int pos0, float *logits, bool all, std::string &err) override {
        return inner_->forward(t, n, pos0, logits, all, err);
    }

private:
    std::unique_ptr<Backend> inner_;
    KvType kv_;
};

// A token list whose pieces decode back to "<id>".
void fill_vocab(Gguf &g, int n_vocab) {
    GgufArray toks;
    toks.reserve(n_vocab);
    for (int i = 0; i < n_vocab; i++) toks.push_back(std::string("<") + std::to_string(i) + ">");
    g.kv["tokenizer.ggml.model"] = std::string("gpt2");
    g.kv["tokenizer.ggml.tokens"] = std::move(toks);
}

// Parses the "<id>" pieces generate() emitted back into ids.
int parse_ids(const std::string &text, int32_t *out, int cap) {
    int n = 0;
    for (size_t i = 0; i < text.size() && n < cap; i++) {
        if (text[i] != '<') continue;
        out[n++] = (int32_t)std::strtol(text.c_str() + i + 1, nullptr, 10);
    }
    return n;
}

}  // namespace

extern "C" {

const char *ts5r_last_error() { return g_err.c_str(); }

float ts5r_fp16_to_fp32(uint16_t h) { return fp16_to_fp32(h); }
uint16_t ts5r_fp32_to_fp16(float f) { return fp32_to_fp16(f); }

int ts5r_dequantize_row(uint32_t type, const void *src, float *dst, int64_t n) {
    try {
        dequantize_row(type, src, dst, n);
    } catch (const std::exception &e) {
        g_err = e.what();
        return -1;
    }
    return 0;
}

// The reference CPU backend over a GGUF file, weights loaded into host memory.
void *ts5r_cpu_open(const char *path, int n_ctx, int kv) {
    auto r = std::make_unique<RefCpu>();
    if (!r->model.open(path, g_err) || !r->model.load(nullptr, g_err)) return nullptr;
    r->backend.reset(make_cpu_backend(r->model, n_ctx, kv_of(kv)));
    return r.release();
}

int ts5r_cpu_forward(void *h, const int32_t *tokens, int n, int pos0, float *logits, int all) {
    RefCpu *r = (RefCpu *)h;
    return r->backend->forward(tokens, n, pos0, logits, all != 0, g_err) ? 0 : -1;
}

int ts5r_cpu_n_vocab(void *h) { return ((RefCpu *)h)->model.hp.n_vocab; }

void ts5r_cpu_close(void *h) { delete (RefCpu *)h; }

// Engine::generate over a table of logits: the ids its sampler picks, with
// speculation off. Returns the count written to out.
int ts5r_sample_table(const float *rows, int n_rows, int n_vocab, float temperature, float top_p, int top_k,
                      uint64_t seed, int max_tokens, int32_t *out) {
    Gguf g;
    fill_vocab(g, n_vocab);
    Tokenizer tok;
    if (!tok.load(g, g_err)) return -1;
    Model m;
    m.hp.n_vocab = n_vocab;
    Engine eng(m, new TableBackend(rows, n_rows, n_vocab, 1 << 20), tok);
    SampleParams p;
    p.temperature = temperature;
    p.top_p = top_p;
    p.top_k = top_k;
    p.seed = seed;
    p.max_tokens = max_tokens;
    p.draft = 0;
    std::string text;
    GenStats st;
    std::vector<int32_t> prompt{1};
    if (!eng.generate(prompt, p, [&](const std::string &s) { text += s; return true; }, st, g_err)) return -1;
    return parse_ids(text, out, max_tokens);
}

// Engine::generate on the reference CPU backend of a GGUF model (whose token
// list must decode to "<id>"), optionally with a draft model. stats:
// [gen_tokens, drafted, draft_accepted].
int ts5r_generate(const char *path, const char *draft_path, int n_ctx, int kv, const int32_t *prompt, int n_prompt,
                  float temperature, float top_p, int top_k, uint64_t seed, int draft, int max_tokens, int32_t *out,
                  int *stats) {
    Model m, dm;
    if (!m.open(path, g_err) || !m.load(nullptr, g_err)) return -1;
    Tokenizer tok;
    if (!tok.load(m.gguf, g_err)) return -1;
    Engine eng(m, make_cpu_backend(m, n_ctx, kv_of(kv)), tok);
    if (draft_path && *draft_path) {
        if (!dm.open(draft_path, g_err) || !dm.load(nullptr, g_err)) return -1;
        if (!eng.set_drafter(dm, make_cpu_backend(dm, n_ctx, kv_of(kv)), g_err)) return -1;
    }
    SampleParams p;
    p.temperature = temperature;
    p.top_p = top_p;
    p.top_k = top_k;
    p.seed = seed;
    p.max_tokens = max_tokens;
    p.draft = draft;
    std::string text;
    GenStats st;
    std::vector<int32_t> pr(prompt, prompt + n_prompt);
    if (!eng.generate(pr, p, [&](const std::string &s) { text += s; return true; }, st, g_err)) return -1;
    if (stats) {
        stats[0] = st.gen_tokens;
        stats[1] = st.drafted;
        stats[2] = st.draft_accepted;
    }
    return parse_ids(text, out, max_tokens);
}

// ts5 check (run_check, engine/src/checks.cpp) of a GGUF model with the CPU
// backend in the GPU's place: it writes the reference's logits for the n test
// tokens next to the model (MODEL.gguf[.q8].ts5ref) as the reference saves
// them. res: max_diff, rel, worst, same_top, pass.
int ts5r_check(const char *path, int kv, int n, double *res) {
    Model m;
    if (!m.open(path, g_err) || !m.load(nullptr, g_err)) return -1;
    KvTagged b(make_cpu_backend(m, n, kv_of(kv)), kv_of(kv));
    CheckResult r;
    if (!run_check(m, b, n, r, g_err, nullptr, true)) return -1;
    res[0] = r.max_diff, res[1] = r.rel, res[2] = r.worst, res[3] = r.same_top, res[4] = r.pass;
    return 0;
}

}  // extern "C"
