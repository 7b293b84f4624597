// A GGUF file into a model in HBM: what ts5 does in Model::open / load
// (engine/src/model.cpp:13-138) followed by the Vulkan backend's weight upload
// and KV sizing (engine/src/vk_backend.cpp:531-600, :620-648, :1364-1402),
// for this backend.
//
//  * The file is parsed here: GGUF v2/v3 header, typed metadata, tensor infos,
//    the data section at general.alignment (default 32).
//  * Hyperparameters come from the architecture's keys with the reference's
//    defaults and its training-context corrections (model.cpp:13-68).
//  * With n_ctx 0 the context is what fits in the device's free memory beside
//    the weights and activations (fit_context), at most the training context;
//    a q8 request gets an f16 cache when the f16 context reaches the training
//    context (f16_reaches), as the reference's Vulkan backend decides.
//  * Upload: worker threads pread whole-row slices of the tensors into pinned
//    staging buffers while another worker's slice goes to HBM on the
//    context's stream (Q6_K / Q8_0 repacked to their split layout there), so
//    the disk, PCIe and the GPU overlap; device calls are serialised.
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "common_host.h"
#include "runtime.h"

using namespace ts5hip;

namespace {

// ---- the file -------------------------------------------------------------------
enum : uint32_t { G_U8, G_I8, G_U16, G_I16, G_U32, G_I32, G_F32, G_BOOL, G_STR, G_ARR, G_U64, G_I64, G_F64 };

struct Meta {
    uint32_t type = 0;
    int64_t i = 0;     // integer and bool values
    double f = 0;      // float values
    std::string s;     // string values
    uint64_t n = 0;    // array length
};

struct TensorInfo {
    std::string name;
    uint32_t type = 0;
    int n_dims = 0;
    int64_t ne[4] = {1, 1, 1, 1};
    uint64_t offset = 0;  // from the data section
};

struct GgufFile {
    std::map<std::string, Meta> kv;
    std::vector<TensorInfo> tensors;
    uint64_t data_offset = 0, file_size = 0;

    const Meta *get(const std::string &k) const {
        auto it = kv.find(k);
        return it == kv.end() ? nullptr : &it->second;
    }
    int64_t num(const std::string &k, int64_t def) const {
        const Meta *m = get(k);
        if (!m) return def;
        return m->type == G_F32 || m->type == G_F64 ? (int64_t)m->f : m->i;
    }
    double real(const std::string &k, double def) const {
        const Meta *m = get(k);
        if (!m) return def;
        return m->type == G_F32 || m->type == G_F64 ? m->f : (double)m->i;
    }
    std::string str(const std::string &k) const {
        const Meta *m = get(k);
        return m && m->type == G_STR ? m->s : std::string();
    }
    const TensorInfo *find(const std::string &name) const {
        for (const TensorInfo &t : tensors)
            if (t.name == name) return &t;
        return nullptr;
    }
};

// Sequential little-endian reads with a sticky failure flag.
struct In {
    FILE *f;
    bool ok = true;
    template <class T>
    T get() {
        T v{};
        if (ok && std::fread(&v, sizeof v, 1, f) != 1) ok = false;
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!ok || n > (1ull << 30)) {
            ok = false;
            return {};
        }
        std::string s((size_t)n, '\0');
        if (n && std::fread(&s[0], 1, (size_t)n, f) != n) ok = false;
        return s;
    }
    void skip(uint64_t bytes) {
        if (ok && fseeko(f, (off_t)bytes, SEEK_CUR) != 0) ok = false;
    }
};

size_t scalar_bytes(uint32_t t) {
    switch (t) {
    case G_U8: case G_I8: case G_BOOL: return 1;
    case G_U16: case G_I16: return 2;
    case G_U32: case G_I32: case G_F32: return 4;
    case G_U64: case G_I64: case G_F64: return 8;
    }
    return 0;
}

bool read_scalar(In &in, uint32_t t, Meta &m) {
    switch (t) {
    case G_U8: m.i = in.get<uint8_t>(); break;
    case G_I8: m.i = in.get<int8_t>(); break;
    case G_U16: m.i = in.get<uint16_t>(); break;
    case G_I16: m.i = in.get<int16_t>(); break;
    case G_U32: m.i = in.get<uint32_t>(); break;
    case G_I32: m.i = in.get<int32_t>(); break;
    case G_U64: m.i = (int64_t)in.get<uint64_t>(); break;
    case G_I64: m.i = in.get<int64_t>(); break;
    case G_BOOL: m.i = in.get<uint8_t>() != 0; break;
    case G_F32: m.f = in.get<float>(); break;
    case G_F64: m.f = in.get<double>(); break;
    case G_STR: m.s = in.str(); break;
    default: return false;
    }
    return in.ok;
}

bool parse(const char *path, GgufFile &g, std::string &err) {
    FILE *f = std::fopen(path, "rb");
    if (!f) {
        err = std::string("cannot open ") + path;
        return false;
    }
    In in{f};
    char magic[4] = {0, 0, 0, 0};
    if (std::fread(magic, 1, 4, f) != 4 || std::memcmp(magic, "GGUF", 4) != 0) {
        std::fclose(f);
        err = std::string(path) + ": not a GGUF file";
        return false;
    }
    const uint32_t version = in.get<uint32_t>();
    const uint64_t n_tensors = in.get<uint64_t>(), n_kv = in.get<uint64_t>();
    if (!in.ok || version < 2 || version > 3 || n_tensors > (1u << 20) || n_kv > (1u << 20)) {
        std::fclose(f);
        err = std::string(path) + ": unsupported GGUF header (version " + std::to_string(version) + ")";
        return false;
    }
    for (uint64_t k = 0; k < n_kv && in.ok; k++) {
        const std::string key = in.str();
        Meta m;
        m.type = in.get<uint32_t>();
        if (m.type == G_ARR) {
            const uint32_t et = in.get<uint32_t>();
            m.n = in.get<uint64_t>();
            if (et == G_STR) {
                for (uint64_t i = 0; i < m.n && in.ok; i++) in.skip(in.get<uint64_t>());
            } else if (scalar_bytes(et)) {
                in.skip(m.n * scalar_bytes(et));
            } else {
                in.ok = false;  // nested arrays: not used by any key the loader reads
            }
        } else if (!read_scalar(in, m.type, m)) {
            in.ok = false;
        }
        g.kv[key] = m;
    }
    g.tensors.resize(n_tensors);
    for (uint64_t k = 0; k < n_tensors && in.ok; k++) {
        TensorInfo &t = g.tensors[k];
        t.name = in.str();
        t.n_dims = (int)in.get<uint32_t>();
        if (t.n_dims < 1 || t.n_dims > 4) in.ok = false;
        for (int d = 0; d < t.n_dims && in.ok; d++) t.ne[d] = (int64_t)in.get<uint64_t>();
        t.type = in.get<uint32_t>();
        t.offset = in.get<uint64_t>();
    }
    const off_t header_end = ftello(f);
    fseeko(f, 0, SEEK_END);
    g.file_size = (uint64_t)ftello(f);
    std::fclose(f);
    if (!in.ok || header_end < 0) {
        err = std::string(path) + ": truncated or malformed GGUF metadata";
        return false;
    }
    const uint64_t align = (uint64_t)std::max<int64_t>(1, g.num("general.alignment", 32));
    g.data_offset = ((uint64_t)header_end + align - 1) / align * align;
    for (const TensorInfo &t : g.tensors) {
        const int bv = block_values(t.type);
        if (bv == 0 || t.ne[0] % bv) continue;  // unsupported types are refused when bound
        const uint64_t bytes = (uint64_t)(t.ne[0] / bv) * gguf_block_bytes(t.type) * t.ne[1] * t.ne[2] * t.ne[3];
        if (g.data_offset + t.offset + bytes > g.file_size) {
            err = std::string(path) + ": tensor " + t.name + " runs past the end of the file";
            return false;
        }
    }
    return true;
}

// Hyperparameters as engine/src/model.cpp:13-68 derives them.
bool hparams_of(const GgufFile &g, ts5hip_hparams &hp, int &n_ctx_train, std::string &err) {
    const std::string arch = g.str("general.architecture");
    if (arch != "llama" && arch != "mistral" && arch != "qwen2" && arch != "qwen3" && arch != "gemma3") {
        err = "architecture '" + arch + "' is not supported";
        return false;
    }
    const std::string a = arch + ".";
    hp = ts5hip_hparams{};
    hp.n_embd = (int)g.num(a + "embedding_length", 0);
    hp.n_layer = (int)g.num(a + "block_count", 0);
    hp.n_ff = (int)g.num(a + "feed_forward_length", 0);
    hp.n_head = (int)g.num(a + "attention.head_count", 0);
    hp.n_head_kv = (int)g.num(a + "attention.head_count_kv", hp.n_head);
    hp.head_dim = (int)g.num(a + "attention.key_length", hp.n_head ? hp.n_embd / hp.n_head : 0);
    n_ctx_train = (int)g.num(a + "context_length", 4096);
    // A context stretched by RoPE scaling the engine does not apply: the
    // original window; Qwen 2.5's files declare 131072 with no scaling keys.
    const std::string scaling = g.str(a + "rope.scaling.type");
    const int original = (int)g.num(a + "rope.scaling.original_context_length", 0);
    if (!scaling.empty() && scaling != "none" && original > 0 && original < n_ctx_train) n_ctx_train = original;
    else if (arch == "qwen2" && scaling.empty() && n_ctx_train > 32768) n_ctx_train = 32768;
    hp.rms_eps = (float)g.real(a + "attention.layer_norm_rms_epsilon", 1e-6);
    hp.rope_base = (float)g.real(a + "rope.freq_base", 10000.0);
    hp.rope_dims = (int)g.num(a + "rope.dimension_count", hp.head_dim);
    hp.rope_neox = arch == "qwen2" || arch == "qwen3" || arch == "gemma3";
    hp.rope_scale = 1.0f;
    if (!hp.n_embd || !hp.n_layer || !hp.n_ff || !hp.n_head) {
        err = "missing hyperparameters";
        return false;
    }
    hp.attn_scale = 1.0f / std::sqrt((float)hp.head_dim);
    if (arch == "gemma3") {
        // What the file does not say, as llama.cpp and the reference fix it:
        // a window on five layers of six with RoPE base 10000 there, the
        // scaled embedding, GELU, and the 27B's (62 layers) query scale.
        hp.embd_scale = std::sqrt((float)hp.n_embd);
        hp.gelu = 1;
        hp.swa_window = (int)g.num(a + "attention.sliding_window", 0);
        hp.swa_pattern = 6;
        hp.rope_base_swa = 10000.f;
        if (scaling == "linear") {
            const double factor = g.real(a + "rope.scaling.factor", 1.0);
            if (factor > 0) hp.rope_scale = (float)(1.0 / factor);
        }
        if (hp.n_layer == 62) hp.attn_scale = 1.0f / std::sqrt((float)(hp.n_embd / hp.n_head));
        // Tests: a small window, so that a short check crosses it (TS5_SWA_WINDOW).
        if (const char *e = std::getenv("TS5_SWA_WINDOW"))
            if (std::atoi(e) > 0 && hp.swa_window > 0) hp.swa_window = std::atoi(e);
        // Gemma 3 layers need their norms after attention and the FFN (model.cpp:114-116).
        for (int l = 0; l < hp.n_layer; l++)
            for (const char *r : {"post_attention_norm.weight", "post_ffw_norm.weight"}) {
                const std::string n = "blk." + std::to_string(l) + "." + r;
                if (!g.find(n)) {
                    err = "missing tensor " + n;
                    return false;
                }
            }
    }
    const TensorInfo *emb = g.find("token_embd.weight");
    if (!emb) {
        err = "missing tensor token_embd.weight";
        return false;
    }
    hp.n_vocab = (int)emb->ne[1];
    return true;
}

// Bytes the model takes in HBM besides its KV cache: the weights in their HBM
// layouts, the single-token buffers, and the 256-token batch buffers with the
// logits rows.
uint64_t fixed_bytes(const GgufFile &g, const ts5hip_hparams &hp) {
    uint64_t w = 0;
    for (const TensorInfo &t : g.tensors) {
        const int64_t rows = t.ne[1] * t.ne[2] * t.ne[3];
        const size_t db = device_bytes(t.type, t.ne[0], rows);
        w += db ? db : (uint64_t)t.ne[0] * rows * 4;
    }
    const uint64_t T = 256, E = hp.n_embd, F = hp.n_ff, QR = (uint64_t)(hp.n_head + 2 * hp.n_head_kv) * hp.head_dim;
    const uint64_t act = 4 * T * (2 * E + QR + 2ull * hp.n_head * hp.head_dim + F) + 2 * 4 * T * hp.n_vocab;
    return w + act + (256ull << 20);  // plus scratch: matmul partials, attention partials, top-k
}

}  // namespace

extern "C" {

uint64_t ts5hip_kv_bytes_per_token(const ts5hip_hparams *hp, int kv_type) {
    if (!hp) return 0;
    const uint64_t values = 2ull * hp->n_layer * hp->n_head_kv * hp->head_dim;  // K and V of every layer
    return kv_type == KV_Q8 ? values + values / 16 : kv_type == KV_F16 ? 2 * values : 4 * values;
}

int ts5hip_fit_context(uint64_t memory, uint64_t used, uint64_t per_token, int cap) {
    const uint64_t reserve = 1ull << 30;  // kept free for everything else
    if (per_token == 0 || memory < used + reserve) return 0;
    const uint64_t n = std::min<uint64_t>((memory - used - reserve) / per_token, cap > 0 ? (uint64_t)cap : 0);
    return (int)(n / 1024 * 1024);
}

int ts5hip_f16_reaches(int f16_ctx, int train) { return train >= 1024 && f16_ctx >= train / 1024 * 1024; }

int ts5hip_gguf_hparams(const char *path, ts5hip_hparams *hp, int *n_ctx_train, int64_t *fixed) {
    if (!path || !hp) return fail(nullptr, TS5HIP_ERR_ARG, "null argument");
    GgufFile g;
    std::string err;
    int train = 0;
    if (!parse(path, g, err) || !hparams_of(g, *hp, train, err)) return fail(nullptr, TS5HIP_ERR_ARG, "%s", err.c_str());
    if (n_ctx_train) *n_ctx_train = train;
    if (fixed) *fixed = (int64_t)fixed_bytes(g, *hp);
    return TS5HIP_OK;
}

int ts5hip_model_load(ts5hip_ctx *ctx, const char *path, int n_ctx, int kv_type, int threads, ts5hip_model **out,
                      int *kv_type_out) {
    if (!ctx || !path || !out) return fail(ctx, TS5HIP_ERR_ARG, "null argument");
    *out = nullptr;
    if (kv_type != KV_Q8 && kv_type != KV_F16)
        return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "KV type %d (the GPU cache is q8 or f16)", kv_type);
    GgufFile g;
    ts5hip_hparams hp;
    std::string err;
    int train = 0;
    if (!parse(path, g, err) || !hparams_of(g, hp, train, err)) return fail(ctx, TS5HIP_ERR_ARG, "%s", err.c_str());
    for (const TensorInfo &t : g.tensors) {
        const bool vec = t.n_dims == 1 || t.ne[1] == 1;
        if (!vec && !ts5hip_supports_type(t.type) && !(t.name == "token_embd.weight" && (t.type == T_F32 || t.type == T_F16)))
            return fail(ctx, TS5HIP_ERR_UNSUPPORTED, "%s: type %u has no kernels here", t.name.c_str(), t.type);
    }
    if (n_ctx <= 0) {
        // As much as fits, at most the training context; q8 becomes f16 when
        // f16 already holds the whole training context (the more exact).
        size_t free_b = 0, total_b = 0;
        TS5_HIP(ctx, hipSetDevice(ctx->device));
        TS5_HIP(ctx, hipMemGetInfo(&free_b, &total_b));
        const int cap = train > 0 ? train : 32768;
        const uint64_t used = fixed_bytes(g, hp);
        const int f16 = ts5hip_fit_context(free_b, used, ts5hip_kv_bytes_per_token(&hp, KV_F16), cap);
        if (kv_type == KV_Q8 && ts5hip_f16_reaches(f16, cap)) kv_type = KV_F16;
        n_ctx = kv_type == KV_F16 ? f16 : ts5hip_fit_context(free_b, used, ts5hip_kv_bytes_per_token(&hp, KV_Q8), cap);
        if (n_ctx <= 0) return fail(ctx, TS5HIP_ERR_CONTEXT_FULL, "not enough GPU memory left for a context of 1024 tokens");
    }
    ts5hip_model *m = nullptr;
    if (int rc = ts5hip_model_create(ctx, &hp, n_ctx, kv_type, &m)) return rc;

    // Work items: every tensor whole, matrices in slices of whole rows.
    struct Item {
        const TensorInfo *t;
        int64_t row0, nrows;
    };
    const size_t SLICE = 64ull << 20;
    std::vector<Item> items;
    for (const TensorInfo &t : g.tensors) {
        const int bv = block_values(t.type);
        if (bv == 0) continue;
        const int64_t rows = t.ne[1] * t.ne[2] * t.ne[3];
        const uint64_t rb = (uint64_t)(t.ne[0] / bv) * gguf_block_bytes(t.type);
        const bool vec = t.n_dims == 1 || rows == 1;
        const int64_t per = vec ? rows : std::max<int64_t>(1, (int64_t)(SLICE / std::max<uint64_t>(rb, 1)));
        for (int64_t r = 0; r < rows; r += per) items.push_back(Item{&t, r, std::min(per, rows - r)});
    }
    const int nthreads = std::max(1, std::min(threads > 0 ? threads : 4, 16));
    std::atomic<size_t> next{0};
    std::atomic<bool> failed{false};
    std::mutex dev_mu;
    int first_rc = TS5HIP_OK;
    std::string first_err;
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) {
        ts5hip_model_destroy(m);
        return fail(ctx, TS5HIP_ERR_ARG, "cannot open %s", path);
    }
    auto worker = [&]() {
        (void)hipSetDevice(ctx->device);  // the current device is per thread
        void *stage = nullptr;
        size_t cap = 0;
        auto fail_once = [&](int rc, const std::string &msg) {
            std::lock_guard<std::mutex> lock(dev_mu);
            if (!failed.exchange(true)) first_rc = rc, first_err = msg;
        };
        for (size_t k; !failed && (k = next.fetch_add(1)) < items.size();) {
            const Item &it = items[k];
            const TensorInfo &t = *it.t;
            const int bv = block_values(t.type);
            const uint64_t rb = (uint64_t)(t.ne[0] / bv) * gguf_block_bytes(t.type);
            const size_t bytes = (size_t)(rb * it.nrows);
            if (bytes > cap) {
                std::lock_guard<std::mutex> lock(dev_mu);
                if (stage) (void)hipHostFree(stage);
                stage = nullptr;
                cap = 0;
                if (hipHostMalloc(&stage, std::max(bytes, SLICE), hipHostMallocDefault) != hipSuccess) {
                    failed = true, first_rc = TS5HIP_ERR_HIP, first_err = "pinned staging buffer";
                    break;
                }
                cap = std::max(bytes, SLICE);
            }
            const uint64_t at = g.data_offset + t.offset + rb * it.row0;
            size_t done = 0;
            while (done < bytes) {
                const ssize_t got = ::pread(fd, (uint8_t *)stage + done, bytes - done, (off_t)(at + done));
                if (got <= 0) break;
                done += (size_t)got;
            }
            if (done != bytes) {
                fail_once(TS5HIP_ERR_ARG, "short read of " + t.name);
                break;
            }
            std::lock_guard<std::mutex> lock(dev_mu);
            if (failed) break;
            const int64_t ne1 = t.ne[1] * t.ne[2] * t.ne[3];
            const int rc = ts5hip_model_set_tensor_rows(m, t.name.c_str(), t.type, t.ne[0], ne1, it.row0, it.nrows,
                                                        stage);
            if (rc != TS5HIP_OK) failed = true, first_rc = rc, first_err = ts5hip_last_error(ctx);
        }
        if (stage) {
            std::lock_guard<std::mutex> lock(dev_mu);
            (void)hipHostFree(stage);
        }
    };
    std::vector<std::thread> pool;
    for (int i = 1; i < nthreads; i++) pool.emplace_back(worker);
    worker();
    for (std::thread &th : pool) th.join();
    ::close(fd);
    if (failed) {
        ts5hip_model_destroy(m);
        return fail(ctx, first_rc, "%s: %s", path, first_err.c_str());
    }
    if (kv_type_out) *kv_type_out = kv_type;
    *out = m;
    return TS5HIP_OK;
}

}  // extern "C"
