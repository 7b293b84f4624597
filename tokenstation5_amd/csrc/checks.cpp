// `ts5 check` over this backend (engine/src/checks.cpp:108-160): the model's
// logits for the check's test tokens against reference logits of ts5's CPU
// backend, with the reference's schedule and bars, and the reference's
// `.ts5ref` files of saved reference logits (engine/src/checks.cpp:28-104),
// read and written in its format so that files from either side serve both.
//
// This library has no CPU backend: the reference logits come from the caller
// (ts5's CpuBackend, or a file saved by an earlier `ts5 check`).
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "common_host.h"
#include "runtime.h"

using namespace ts5hip;

namespace {

// The .ts5ref header (the reference's RefHeader layout, 40 bytes): magic,
// format version, positions, vocabulary, cache code (0 f16, 1 q8, 2 f32),
// then the model file's size and the FNV-1a hash of its first MiB.
struct RefFileHeader {
    char magic[8];
    uint32_t version, n, n_vocab, kv;
    uint64_t file_size, file_hash;
};
static_assert(sizeof(RefFileHeader) == 40, ".ts5ref header layout");
constexpr uint32_t kRefFormat = 1;

uint32_t cache_code(int kv_type) { return kv_type == KV_F16 ? 0u : kv_type == KV_Q8 ? 1u : 2u; }

std::string ref_file(const std::string &model, int kv_type) {
    const char *tag = kv_type == KV_F16 ? "" : kv_type == KV_Q8 ? ".q8" : ".f32";
    return model + tag + ".ts5ref";
}

bool header_for(const char *model, int n, int n_vocab, int kv_type, RefFileHeader &h) {
    std::memset(&h, 0, sizeof h);
    std::memcpy(h.magic, "TS5REF\0\0", 8);
    h.version = kRefFormat, h.n = (uint32_t)n, h.n_vocab = (uint32_t)n_vocab, h.kv = cache_code(kv_type);
    return ts5hip_model_file_id(model, &h.file_size, &h.file_hash) == TS5HIP_OK;
}

double ms_since(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

}  // namespace

extern "C" {

int ts5hip_check_tokens(int n, int n_vocab, int32_t *out) {
    if (!out || n <= 0 || n_vocab <= 1000) return fail(nullptr, TS5HIP_ERR_ARG, "check tokens need n_vocab > 1000");
    for (int i = 0; i < n; i++) out[i] = 1000 + (int32_t)(((int64_t)i * 7919) % (n_vocab - 1000));
    return TS5HIP_OK;
}

int ts5hip_model_file_id(const char *path, uint64_t *size, uint64_t *hash) {
    if (!path || !size || !hash) return fail(nullptr, TS5HIP_ERR_ARG, "null argument");
    FILE *f = std::fopen(path, "rb");
    if (!f) return fail(nullptr, TS5HIP_ERR_ARG, "cannot open %s", path);
    std::vector<unsigned char> head(1 << 20);
    const size_t got = std::fread(head.data(), 1, head.size(), f);
    fseeko(f, 0, SEEK_END);
    *size = (uint64_t)ftello(f);
    std::fclose(f);
    uint64_t h = 1469598103934665603ull;  // FNV-1a over the first MiB
    for (size_t i = 0; i < got; i++) h = (h ^ head[i]) * 1099511628211ull;
    *hash = h;
    return TS5HIP_OK;
}

int ts5hip_ref_path(const char *model_path, int kv_type, char *out, int len) {
    if (!model_path || !out || len <= 0) return fail(nullptr, TS5HIP_ERR_ARG, "null argument");
    const std::string p = ref_file(model_path, kv_type);
    if ((int)p.size() >= len) return fail(nullptr, TS5HIP_ERR_ARG, "path buffer of %d bytes", len);
    std::memcpy(out, p.c_str(), p.size() + 1);
    return TS5HIP_OK;
}

int ts5hip_ref_load(const char *model_path, int n, int n_vocab, int kv_type, float *logits) {
    if (!model_path || !logits || n <= 0 || n_vocab <= 0) return fail(nullptr, TS5HIP_ERR_ARG, "bad argument");
    RefFileHeader want, h;
    if (!header_for(model_path, n, n_vocab, kv_type, want)) return fail(nullptr, TS5HIP_ERR_ARG, "cannot read %s", model_path);
    const std::string p = ref_file(model_path, kv_type);
    FILE *f = std::fopen(p.c_str(), "rb");
    if (!f) return fail(nullptr, TS5HIP_ERR_STATE, "no saved reference logits at %s", p.c_str());
    // The saved file must be of this model file and cache type and hold at
    // least n positions; the first n are read.
    const bool same = std::fread(&h, sizeof h, 1, f) == 1 && std::memcmp(h.magic, want.magic, 8) == 0 &&
                      h.version == want.version && h.n >= want.n && h.n_vocab == want.n_vocab && h.kv == want.kv &&
                      h.file_size == want.file_size && h.file_hash == want.file_hash;
    const size_t count = (size_t)n * n_vocab;
    const bool ok = same && std::fread(logits, 4, count, f) == count;
    std::fclose(f);
    if (!ok) return fail(nullptr, TS5HIP_ERR_STATE, "%s is not for this model, cache type and %d positions", p.c_str(), n);
    return TS5HIP_OK;
}

int ts5hip_ref_save(const char *model_path, int n, int n_vocab, int kv_type, const float *logits) {
    if (!model_path || !logits || n <= 0 || n_vocab <= 0) return fail(nullptr, TS5HIP_ERR_ARG, "bad argument");
    const std::string p = ref_file(model_path, kv_type), part = p + ".part";
    // A file of the same format and cache type with more positions is kept.
    if (FILE *f = std::fopen(p.c_str(), "rb")) {
        RefFileHeader h;
        const bool more = std::fread(&h, sizeof h, 1, f) == 1 && h.version == kRefFormat &&
                          h.kv == cache_code(kv_type) && (int)h.n > n;
        std::fclose(f);
        if (more) return TS5HIP_OK;
    }
    RefFileHeader h;
    if (!header_for(model_path, n, n_vocab, kv_type, h)) return fail(nullptr, TS5HIP_ERR_ARG, "cannot read %s", model_path);
    FILE *f = std::fopen(part.c_str(), "wb");
    const size_t count = (size_t)n * n_vocab;
    bool ok = f && std::fwrite(&h, sizeof h, 1, f) == 1 && std::fwrite(logits, 4, count, f) == count;
    if (f) ok = std::fclose(f) == 0 && ok;
    if (ok) ok = std::rename(part.c_str(), p.c_str()) == 0;
    if (!ok) {
        std::remove(part.c_str());
        return fail(nullptr, TS5HIP_ERR_ARG, "cannot write %s", p.c_str());
    }
    return TS5HIP_OK;
}

int ts5hip_check_run(ts5hip_model *m, const char *model_path, int n, const float *ref_logits, ts5hip_check_result *r) {
    ts5hip_ctx *ctx = m ? model_ctx(m) : nullptr;
    if (!m || !r || n < 2) return fail(ctx, TS5HIP_ERR_ARG, "bad argument");
    if (n > ts5hip_n_ctx(m)) return fail(ctx, TS5HIP_ERR_CONTEXT_FULL, "a check of %d tokens in a context of %d", n, ts5hip_n_ctx(m));
    const int nv = model_vocab(m), kv = ts5hip_kv_type(m);
    std::memset(r, 0, sizeof *r);
    r->n = n;
    std::vector<int32_t> toks((size_t)n);
    if (int rc = ts5hip_check_tokens(n, nv, toks.data())) return fail(ctx, rc, "%s", ts5hip_last_error(nullptr));
    std::vector<float> ref;
    if (!ref_logits) {
        if (!model_path) return fail(ctx, TS5HIP_ERR_ARG, "no reference logits and no model file");
        ref.resize((size_t)n * nv);
        if (int rc = ts5hip_ref_load(model_path, n, nv, kv, ref.data()))
            return fail(ctx, rc, "%s", ts5hip_last_error(nullptr));
        ref_logits = ref.data();
        r->saved = 1;
    }
    // The prompt's way for most positions (one call, every position's
    // logits), then generation's for the last few: one token per call.
    std::vector<float> got((size_t)n * nv);
    const int single = std::min(4, n / 2), batch = n - single;
    const auto t0 = std::chrono::steady_clock::now();
    if (int rc = ts5hip_forward(m, toks.data(), batch, 0, got.data(), 1)) return rc;
    for (int i = batch; i < n; i++)
        if (int rc = ts5hip_forward(m, &toks[(size_t)i], 1, i, got.data() + (size_t)i * nv, 0)) return rc;
    r->gpu_ms = ms_since(t0);
    double max_ref = 0;
    for (int i = 0; i < n; i++) {
        const float *g = got.data() + (size_t)i * nv, *f = ref_logits + (size_t)i * nv;
        for (int j = 0; j < nv; j++) {
            const double d = std::fabs((double)g[j] - (double)f[j]);
            if (d > r->max_diff) r->max_diff = d, r->worst = i;
            max_ref = std::max(max_ref, (double)std::fabs(f[j]));
        }
        r->same_top += (std::max_element(g, g + nv) - g) == (std::max_element(f, f + nv) - f);
    }
    r->rel = max_ref > 0 ? r->max_diff / max_ref : r->max_diff;
    // The reference's bars: 0.5 % of the largest logit, 2 % with an 8-bit
    // cache (whose rounding steps differ wherever the two sides' inputs do).
    r->pass = std::isfinite(r->rel) && r->rel < (kv == KV_Q8 ? 2e-2 : 5e-3);
    return TS5HIP_OK;
}

}  // extern "C"
