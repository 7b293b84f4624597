// The `ts5 check` harness over this backend, and its saved reference logits.
//
// What has to agree with ts5 is data and policy, which this file states once:
//  * a .ts5ref file is a 40-byte little-endian header followed by
//    positions x vocabulary fp32 logits. The header: the 8 bytes "TS5REF\0\0",
//    then u32 format (1), positions, vocabulary and cache code (0 f16, 1 q8,
//    2 f32), then u64 byte size of the model file and an FNV-1a style 64-bit
//    hash of its first MiB (engine/src/checks.cpp:28-50);
//  * it lives beside the model as MODEL.ts5ref (f16 cache), MODEL.q8.ts5ref or
//    MODEL.f32.ts5ref (engine/src/checks.cpp:53-58);
//  * the check feeds the tokens 1000 + (7919 i mod (n_vocab - 1000)), the first
//    n - min(4, n/2) as one prompt with every position's logits, the rest one
//    token per call, and passes when the largest |difference| is under 0.5 % of
//    the largest |reference logit|, 2 % with a q8 cache
//    (engine/src/checks.cpp:22-26, :108-160).
// Files written here and files ts5 writes are interchangeable.
//
// This library has no CPU backend: the reference logits come from the caller
// (ts5's CpuBackend, or a file saved by either side).
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstring>
#include <string>
#include <vector>

#include "common_host.h"
#include "runtime.h"

using namespace ts5hip;

namespace {

constexpr size_t kHeaderBytes = 40;
constexpr uint8_t kMagic[8] = {'T', 'S', '5', 'R', 'E', 'F', 0, 0};
constexpr uint32_t kFormat = 1;
constexpr size_t kIdentityBytes = size_t(1) << 20;  // the model file's hashed prefix

uint32_t cache_code(int kv_type) { return kv_type == KV_F16 ? 0u : kv_type == KV_Q8 ? 1u : 2u; }

const char *cache_suffix(int kv_type) { return kv_type == KV_F16 ? ".ts5ref" : kv_type == KV_Q8 ? ".q8.ts5ref" : ".f32.ts5ref"; }

// The header's fields after the magic, with an explicit little-endian codec.
struct RefHeader {
    uint32_t format = kFormat, positions = 0, vocab = 0, cache = 0;
    uint64_t model_size = 0, model_hash = 0;

    void encode(uint8_t *out) const {
        auto put = [&out](uint64_t v, int bytes) {
            for (int i = 0; i < bytes; i++) *out++ = uint8_t(v >> (8 * i));
        };
        std::memcpy(out, kMagic, sizeof kMagic);
        out += sizeof kMagic;
        put(format, 4), put(positions, 4), put(vocab, 4), put(cache, 4);
        put(model_size, 8), put(model_hash, 8);
    }
    // False when the bytes are not a .ts5ref header at all.
    bool decode(const uint8_t *in) {
        if (std::memcmp(in, kMagic, sizeof kMagic) != 0) return false;
        in += sizeof kMagic;
        auto get = [&in](int bytes) {
            uint64_t v = 0;
            for (int i = bytes - 1; i >= 0; i--) v = v << 8 | in[i];
            in += bytes;
            return v;
        };
        format = (uint32_t)get(4), positions = (uint32_t)get(4), vocab = (uint32_t)get(4), cache = (uint32_t)get(4);
        model_size = get(8), model_hash = get(8);
        return true;
    }
    // Why a saved header cannot serve a request for `want` (nullptr: it can).
    const char *unfit_for(const RefHeader &want) const {
        if (format != want.format) return "another format version";
        if (cache != want.cache) return "another cache type";
        if (model_size != want.model_size || model_hash != want.model_hash) return "another model file";
        if (vocab != want.vocab) return "another vocabulary";
        if (positions < want.positions) return "fewer positions";
        return nullptr;
    }
};

// A file descriptor closed when it goes out of scope.
class Fd {
  public:
    explicit Fd(int fd) : fd_(fd) {}
    ~Fd() {
        if (fd_ >= 0) ::close(fd_);
    }
    Fd(const Fd &) = delete;
    Fd &operator=(const Fd &) = delete;
    int get() const { return fd_; }
    bool open() const { return fd_ >= 0; }
    // Closes now and reports whether the close (the last chance of a write error) succeeded.
    bool close_checked() {
        const int fd = fd_;
        fd_ = -1;
        return fd >= 0 && ::close(fd) == 0;
    }

  private:
    int fd_;
};

// pread/write until every byte is through (short transfers and EINTR retried).
bool read_at(int fd, void *dst, size_t len, off_t at) {
    auto *p = static_cast<uint8_t *>(dst);
    while (len > 0) {
        const ssize_t got = ::pread(fd, p, len, at);
        if (got < 0 && errno == EINTR) continue;
        if (got <= 0) return false;
        p += got, len -= (size_t)got, at += got;
    }
    return true;
}

bool write_all(int fd, const void *src, size_t len) {
    auto *p = static_cast<const uint8_t *>(src);
    while (len > 0) {
        const ssize_t put = ::write(fd, p, len);
        if (put < 0 && errno == EINTR) continue;
        if (put <= 0) return false;
        p += put, len -= (size_t)put;
    }
    return true;
}

// The model file's size and the hash of its first MiB, read in 64 KiB pieces.
// The hash is FNV-1a's xor-multiply with the 64-bit FNV prime, started from
// 1469598103934665603: the value ts5 writes (engine/src/checks.cpp:47), which
// is not FNV's published offset basis 14695981039346656037, so files from
// either side carry the same id.
constexpr uint64_t kHashStart = 1469598103934665603ull, kHashPrime = 0x100000001b3ull;

bool model_identity(const char *path, uint64_t &size, uint64_t &hash) {
    Fd f(::open(path, O_RDONLY | O_CLOEXEC));
    struct stat st;
    if (!f.open() || ::fstat(f.get(), &st) != 0) return false;
    size = (uint64_t)st.st_size;
    hash = kHashStart;
    std::vector<uint8_t> piece(64 << 10);
    const size_t span = std::min<uint64_t>(size, kIdentityBytes);
    for (size_t at = 0; at < span;) {
        const size_t len = std::min(piece.size(), span - at);
        if (!read_at(f.get(), piece.data(), len, (off_t)at)) return false;
        for (size_t i = 0; i < len; i++) hash = (hash ^ piece[i]) * kHashPrime;
        at += len;
    }
    return true;
}

// The header a file for this model, request size and cache type carries.
bool header_of(const char *model, int positions, int vocab, int kv_type, RefHeader &h) {
    h = RefHeader{};
    h.positions = (uint32_t)positions, h.vocab = (uint32_t)vocab, h.cache = cache_code(kv_type);
    return model_identity(model, h.model_size, h.model_hash);
}

// The header of an existing .ts5ref file (false: missing, short, or not one).
bool saved_header(const std::string &path, RefHeader &h) {
    Fd f(::open(path.c_str(), O_RDONLY | O_CLOEXEC));
    uint8_t raw[kHeaderBytes];
    return f.open() && read_at(f.get(), raw, sizeof raw, 0) && h.decode(raw);
}

// Writes the pieces to path + ".part", then renames it over path, so a reader
// never sees a half-written file; the partial file is removed on failure.
bool replace_file(const std::string &path, std::initializer_list<std::pair<const void *, size_t>> pieces) {
    const std::string part = path + ".part";
    bool ok;
    {
        Fd f(::open(part.c_str(), O_WRONLY | O_CREAT | O_TRUNC | O_CLOEXEC, 0644));
        ok = f.open();
        for (const auto &pc : pieces) ok = ok && write_all(f.get(), pc.first, pc.second);
        ok = f.close_checked() && ok;
    }
    ok = ok && ::rename(part.c_str(), path.c_str()) == 0;
    if (!ok) ::unlink(part.c_str());
    return ok;
}

// Largest |got - ref| over rows (with its row), largest |ref|, rows whose
// first maximum is at the same index, and whether every got value is finite.
struct Agreement {
    double max_diff = 0, max_ref = 0;
    int worst = 0, same_top = 0;
    bool finite = true;

    static int first_max(const float *v, int n) {
        int best = 0;
        for (int j = 1; j < n; j++)
            if (v[j] > v[best]) best = j;
        return best;
    }
    void add_row(int row, const float *got, const float *ref, int n) {
        for (int j = 0; j < n; j++) {
            finite = finite && std::isfinite(got[j]);
            const double diff = std::fabs((double)got[j] - (double)ref[j]);
            if (diff > max_diff) {
                max_diff = diff;
                worst = row;
            }
            max_ref = std::max(max_ref, std::fabs((double)ref[j]));
        }
        if (first_max(got, n) == first_max(ref, n)) same_top++;
    }
};

}  // namespace

extern "C" {

int ts5hip_check_tokens(int n, int n_vocab, int32_t *out) {
    if (!out || n <= 0 || n_vocab <= 1000) return fail(nullptr, TS5HIP_ERR_ARG, "check tokens need n_vocab > 1000");
    const int64_t span = n_vocab - 1000;
    for (int i = 0; i < n; i++) out[i] = (int32_t)(1000 + (int64_t)i * 7919 % span);
    return TS5HIP_OK;
}

int ts5hip_model_file_id(const char *path, uint64_t *size, uint64_t *hash) {
    if (!path || !size || !hash) return fail(nullptr, TS5HIP_ERR_ARG, "null argument");
    if (!model_identity(path, *size, *hash)) return fail(nullptr, TS5HIP_ERR_ARG, "cannot read %s", path);
    return TS5HIP_OK;
}

int ts5hip_ref_path(const char *model_path, int kv_type, char *out, int len) {
    if (!model_path || !out || len <= 0) return fail(nullptr, TS5HIP_ERR_ARG, "null argument");
    const std::string p = std::string(model_path) + cache_suffix(kv_type);
    if ((int)p.size() >= len) return fail(nullptr, TS5HIP_ERR_ARG, "path buffer of %d bytes", len);
    std::memcpy(out, p.c_str(), p.size() + 1);
    return TS5HIP_OK;
}

int ts5hip_ref_load(const char *model_path, int n, int n_vocab, int kv_type, float *logits) {
    if (!model_path || !logits || n <= 0 || n_vocab <= 0) return fail(nullptr, TS5HIP_ERR_ARG, "bad argument");
    RefHeader want, have;
    if (!header_of(model_path, n, n_vocab, kv_type, want)) return fail(nullptr, TS5HIP_ERR_ARG, "cannot read %s", model_path);
    const std::string p = std::string(model_path) + cache_suffix(kv_type);
    Fd f(::open(p.c_str(), O_RDONLY | O_CLOEXEC));
    if (!f.open()) return fail(nullptr, TS5HIP_ERR_STATE, "no saved reference logits at %s", p.c_str());
    uint8_t raw[kHeaderBytes];
    if (!read_at(f.get(), raw, sizeof raw, 0) || !have.decode(raw))
        return fail(nullptr, TS5HIP_ERR_STATE, "%s is not a .ts5ref file", p.c_str());
    if (const char *why = have.unfit_for(want))
        return fail(nullptr, TS5HIP_ERR_STATE, "%s is for %s (wanted %d positions of this model and cache)", p.c_str(), why, n);
    // The first n rows; rows past them (a file saved for a longer check) stay unread.
    if (!read_at(f.get(), logits, (size_t)n * n_vocab * sizeof(float), (off_t)kHeaderBytes))
        return fail(nullptr, TS5HIP_ERR_STATE, "%s ends before its %d rows of logits", p.c_str(), n);
    return TS5HIP_OK;
}

int ts5hip_ref_save(const char *model_path, int n, int n_vocab, int kv_type, const float *logits) {
    if (!model_path || !logits || n <= 0 || n_vocab <= 0) return fail(nullptr, TS5HIP_ERR_ARG, "bad argument");
    RefHeader h;
    if (!header_of(model_path, n, n_vocab, kv_type, h)) return fail(nullptr, TS5HIP_ERR_ARG, "cannot read %s", model_path);
    const std::string p = std::string(model_path) + cache_suffix(kv_type);
    // A saved file that already serves a longer check of this model and cache stays.
    RefHeader old;
    if (saved_header(p, old) && old.unfit_for(h) == nullptr && old.positions > h.positions) return TS5HIP_OK;
    uint8_t raw[kHeaderBytes];
    h.encode(raw);
    if (!replace_file(p, {{raw, sizeof raw}, {logits, (size_t)n * n_vocab * sizeof(float)}}))
        return fail(nullptr, TS5HIP_ERR_ARG, "cannot write %s", p.c_str());
    return TS5HIP_OK;
}

int ts5hip_check_run(ts5hip_model *m, const char *model_path, int n, const float *ref_logits, ts5hip_check_result *r) {
    ts5hip_ctx *ctx = m ? model_ctx(m) : nullptr;
    if (!m || !r || n < 2) return fail(ctx, TS5HIP_ERR_ARG, "bad argument");
    if (n > ts5hip_n_ctx(m)) return fail(ctx, TS5HIP_ERR_CONTEXT_FULL, "a check of %d tokens in a context of %d", n, ts5hip_n_ctx(m));
    const int nv = model_vocab(m), kv = ts5hip_kv_type(m);
    *r = ts5hip_check_result{};
    r->n = n;

    std::vector<float> saved;
    if (!ref_logits) {
        if (!model_path) return fail(ctx, TS5HIP_ERR_ARG, "no reference logits and no model file");
        saved.resize((size_t)n * nv);
        if (int rc = ts5hip_ref_load(model_path, n, nv, kv, saved.data())) return fail(ctx, rc, "%s", ts5hip_last_error(nullptr));
        ref_logits = saved.data();
        r->saved = 1;
    }
    std::vector<int32_t> tokens((size_t)n);
    if (int rc = ts5hip_check_tokens(n, nv, tokens.data())) return fail(ctx, rc, "%s", ts5hip_last_error(nullptr));

    // Both ways the engine feeds a backend: a prompt (one call, every row's
    // logits) and then generation (one token a call, its own row).
    struct Call {
        int first, count, every_row;
    };
    const int generated = std::min(4, n / 2);
    std::vector<Call> calls{{0, n - generated, 1}};
    for (int i = n - generated; i < n; i++) calls.push_back({i, 1, 0});

    std::vector<float> logits((size_t)n * nv);
    const auto start = std::chrono::steady_clock::now();
    for (const Call &c : calls)
        if (int rc = ts5hip_forward(m, tokens.data() + c.first, c.count, c.first, logits.data() + (size_t)c.first * nv, c.every_row))
            return rc;
    r->gpu_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - start).count();

    Agreement a;
    for (int i = 0; i < n; i++) a.add_row(i, logits.data() + (size_t)i * nv, ref_logits + (size_t)i * nv, nv);
    r->max_diff = a.max_diff, r->worst = a.worst, r->same_top = a.same_top;
    r->rel = a.max_ref > 0 ? a.max_diff / a.max_ref : a.max_diff;
    // A q8 cache rounds each side's slightly different K/V values to 1/127
    // steps that can land apart, hence its wider bar. Non-finite output fails.
    const double bar = kv == KV_Q8 ? 2e-2 : 5e-3;
    r->pass = a.finite && std::isfinite(r->rel) && r->rel < bar;
    return TS5HIP_OK;
}

}  // extern "C"
