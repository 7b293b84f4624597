// The decode driver over the C ABI: generation with speculative decoding, the
// behaviour of ts5's Engine::generate (engine/src/engine.cpp:149-292).
//
// A generation keeps a history (the token ids whose K/V the target's cache
// holds, position = index) and runs in steps. Each step forwards the pending
// token plus up to `room` drafted continuations as one batch and keeps the
// drafts the target's own sampler reproduces, so the output is the one a
// token-at-a-time loop would give with the same sampler stream. Drafts come
// from two sources, cheapest first:
//   * the history itself: what followed the most recent earlier occurrence
//     of the last three tokens (else two), found by a hash-chain match
//     finder over the history's 2-grams (the prompt-lookup drafting of
//     engine.cpp:134-147);
//   * a draft model (engine.cpp:75-129): its greedy continuation, after
//     catching its own cache up with the history.
// How many tokens to draft follows the recent acceptance rate (engine.cpp:
// 218-228): a running average of accepted / proposed picks full, short or no
// drafts, with a periodic short probe while drafting is off.
//
// Sampling reads no logits row on the host unless it must: every row of a
// step's batch is reduced on the GPU in one pass (greedy argmax, or the top
// k + 1 candidates), and the host draws from those (model_draw).
#include <algorithm>
#include <cstring>
#include <random>
#include <vector>

#include "common_host.h"
#include "runtime.h"

using namespace ts5hip;

namespace {

// Batches of prompt (and draft catch-up) tokens per forward: the reference's
// chunk (engine.cpp:172, :97), which is also the backend's logits capacity.
constexpr int kChunk = 256;

// ---------------------------------------------------------------------------
// Prompt lookup: a match finder over the history. Every 2-gram (h[j-1], h[j])
// is linked into a chain of the positions j that end a 2-gram of the same
// hash, newest first (the hash chains of LZ77 match finders). A lookup for the
// pending token t walks the chain of (h[n-1], t): the first real match whose
// predecessor is also h[n-2] is the newest 3-gram occurrence; failing that the
// first real match is the newest 2-gram one. The drafts are what followed it
// in the history extended by t.
// ---------------------------------------------------------------------------
class MatchFinder {
public:
    void rebuild(const std::vector<int32_t> &h) {
        size_t want = 1024;
        while (want < 2 * h.size() + 2) want <<= 1;
        head_.assign(want, -1);
        mask_ = (uint32_t)(want - 1);
        link_.clear();
        indexed_ = 0;
        extend(h);
    }
    // Links the 2-grams ending at the positions added since the last call.
    void extend(const std::vector<int32_t> &h) {
        if (2 * h.size() + 2 > head_.size()) {
            rebuild(h);
            return;
        }
        link_.resize(h.size(), -1);
        for (size_t j = std::max<size_t>(indexed_, 1); j < h.size(); j++) {
            int32_t &slot = head_[bucket(h[j - 1], h[j])];
            link_[j] = slot;
            slot = (int32_t)j;
        }
        indexed_ = h.size();
    }
    // The position just past the newest match for pending token t, or -1.
    int64_t find(const std::vector<int32_t> &h, int32_t t) const {
        const size_t n = h.size();
        if (n == 0 || head_.empty()) return -1;
        const int32_t a = h[n - 1];
        int64_t newest2 = -1;
        for (int32_t j = head_[bucket(a, t)]; j >= 0; j = link_[(size_t)j]) {
            if (h[(size_t)j - 1] != a || h[(size_t)j] != t) continue;  // another 2-gram of the same hash
            if (newest2 < 0) newest2 = j + 1;
            if (n >= 2 && j >= 2 && h[(size_t)j - 2] == h[n - 2]) return j + 1;
        }
        return newest2;
    }

private:
    uint32_t bucket(int32_t a, int32_t b) const {
        uint64_t x = (uint64_t)(uint32_t)a * 0x9E3779B97F4A7C15ull ^ (uint64_t)(uint32_t)b * 0xC2B2AE3D27D4EB4Full;
        x ^= x >> 29;
        return (uint32_t)(x ^ (x >> 32)) & mask_;
    }
    std::vector<int32_t> head_, link_;
    uint32_t mask_ = 0;
    size_t indexed_ = 0;
};

// ---------------------------------------------------------------------------
// The draft model: its cache holds the first `synced` history positions.
// ---------------------------------------------------------------------------
struct Drafter {
    ts5hip_model *m = nullptr;
    size_t synced = 0;
    bool live = false;  // false once a forward failed or a token fell outside its vocabulary
    RowPicks pick;
    std::vector<int32_t> feed;

    bool all_known(const int32_t *ids, size_t n) {
        const int nv = model_vocab(m);
        for (size_t i = 0; i < n; i++)
            if (ids[i] >= nv) return live = false;
        return true;
    }

    // Up to `room` drafts after pending token t at position h.size(), appended
    // to out. A backlog of a whole chunk or more is caught up by one chunk
    // instead (no drafts this step), so no step stalls on a long prompt.
    void propose(const std::vector<int32_t> &h, int32_t t, int room, int target_vocab, const int32_t *eog,
                 int n_eog, std::vector<int32_t> &out) {
        const size_t pos = h.size();
        if ((int64_t)pos + room + 2 > ts5hip_n_ctx(m)) return;
        if (pos - synced >= (size_t)kChunk) {
            if (!all_known(h.data() + synced, kChunk)) return;
            if (ts5hip_forward(m, h.data() + synced, kChunk, (int)synced, nullptr, 0) != TS5HIP_OK) live = false;
            else synced += kChunk;
            return;
        }
        feed.assign(h.begin() + (ptrdiff_t)synced, h.end());
        feed.push_back(t);
        if (!all_known(feed.data(), feed.size())) return;
        // The first draft is the greedy pick after the catch-up batch; the
        // rest come from the device-side greedy loop in one call (it writes
        // K/V past a stop as well; those positions are re-fed before use).
        if (ts5hip_forward_in_place(m, feed.data(), (int)feed.size(), (int)synced, 0) != TS5HIP_OK ||
            model_pick_rows(m, 0, 1, 0.f, 0, pick) != TS5HIP_OK) {
            live = false;
            return;
        }
        int32_t next[256];
        next[0] = pick.id[0];
        if (room > 1 && next[0] < target_vocab && std::find(eog, eog + n_eog, next[0]) == eog + n_eog &&
            ts5hip_generate_greedy(m, next[0], (int)pos + 1, room - 1, next + 1) != TS5HIP_OK) {
            live = false;
            room = 1;
        }
        for (int i = 0; i < room; i++) {
            if (next[i] >= target_vocab) break;  // a padded drafter row is no target token
            out.push_back(next[i]);
            if (std::find(eog, eog + n_eog, next[i]) != eog + n_eog) break;  // nothing follows an end
        }
    }
};

// ---------------------------------------------------------------------------
// Draft length from the running acceptance rate (engine.cpp:218-228, :270-273):
// below 15 % no drafts (but a short probe every 16th step), below 50 % at most
// 3, else the full length. The average moves a fifth of the way to each
// judged batch's rate.
// ---------------------------------------------------------------------------
class DraftGovernor {
public:
    explicit DraftGovernor(bool adaptive) : adaptive_(adaptive) {}
    int length(int full) {
        int n = full;
        if (adaptive_ && rate_ >= 0) {
            const int shortlen = std::min(full, kShort);
            n = rate_ < kOff ? 0 : rate_ < kHalf ? shortlen : full;
            if (n == 0 && step_ % kProbeEvery == 0) n = shortlen;
        }
        step_++;
        return n;
    }
    void judged(int accepted, int proposed) {
        if (proposed <= 0) return;
        const float r = (float)accepted / (float)proposed;
        rate_ = rate_ < 0 ? r : kKeep * rate_ + kTake * r;
    }

private:
    static constexpr float kOff = 0.15f, kHalf = 0.5f, kKeep = 0.8f, kTake = 0.2f;
    static constexpr int kShort = 3, kProbeEvery = 16;
    bool adaptive_;
    float rate_ = -1;  // < 0 until a batch with drafts has been judged
    int step_ = 0;
};

bool ends(const int32_t *eog, int n_eog, int32_t t) { return std::find(eog, eog + n_eog, t) != eog + n_eog; }

}  // namespace

struct ts5hip_engine {
    ts5hip_model *m = nullptr;
    ts5hip_sampler *rng = nullptr;  // the sampler stream (std::mt19937_64, default-seeded at creation)
    std::vector<int32_t> history;
    MatchFinder finder;
    Drafter drafter;
    RowPicks picks;
    std::vector<int32_t> batch;
    // The last generation's drafts by source: lookup drafted, accepted; model drafted, accepted.
    int32_t by_source[4] = {0, 0, 0, 0};

    void forget() {
        history.clear();
        drafter.synced = 0;
    }
};

extern "C" {

int ts5hip_engine_new(ts5hip_model *m, ts5hip_engine **out) {
    if (!m || !out) return fail(nullptr, TS5HIP_ERR_ARG, "null argument");
    ts5hip_engine *e = new ts5hip_engine();
    e->m = m;
    e->rng = ts5hip_sampler_new(std::mt19937_64::default_seed);
    *out = e;
    return TS5HIP_OK;
}

void ts5hip_engine_free(ts5hip_engine *e) {
    if (!e) return;
    ts5hip_sampler_free(e->rng);
    delete e;
}

int ts5hip_engine_set_drafter(ts5hip_engine *e, ts5hip_model *dm) {
    if (!e) return fail(nullptr, TS5HIP_ERR_ARG, "null engine");
    e->drafter = Drafter{};
    e->drafter.m = dm;
    e->drafter.live = dm != nullptr;
    return TS5HIP_OK;
}

int ts5hip_engine_draft_sources(const ts5hip_engine *e, int32_t *out) {
    if (!e || !out) return fail(nullptr, TS5HIP_ERR_ARG, "null argument");
    std::memcpy(out, e->by_source, sizeof e->by_source);
    return TS5HIP_OK;
}

int ts5hip_engine_drafter_state(const ts5hip_engine *e) {
    if (!e || !e->drafter.m) return 0;
    return e->drafter.live ? 1 : 2;
}

int ts5hip_engine_generate(ts5hip_engine *e, const int32_t *prompt, int n_prompt, const ts5hip_sample_params *p,
                           const int32_t *eog, int n_eog, int32_t *out, int32_t *stats) {
    if (!e || !prompt || !p || !out || (n_eog > 0 && !eog)) return fail(nullptr, TS5HIP_ERR_ARG, "null argument");
    ts5hip_model *m = e->m;
    ts5hip_ctx *ctx = model_ctx(m);
    if (n_prompt <= 0) return fail(ctx, TS5HIP_ERR_ARG, "empty prompt");
    if (n_prompt + 1 > ts5hip_n_ctx(m)) return fail(ctx, TS5HIP_ERR_CONTEXT_FULL, "prompt longer than the context");
    if (p->seed) sampler_reseed(e->rng, p->seed);
    const int n_ctx = ts5hip_n_ctx(m);
    std::vector<int32_t> &h = e->history;
    enum { S_PROMPT, S_EVAL, S_GEN, S_DRAFTED, S_ACCEPTED, S_EOG };
    int32_t st[6] = {n_prompt, 0, 0, 0, 0, 0};
    std::fill(e->by_source, e->by_source + 4, 0);

    // The prompt: the cached history's common prefix is kept, except that the
    // last prompt token is always run (its logits start the generation).
    const size_t common = std::mismatch(h.begin(), h.begin() + std::min(h.size(), (size_t)n_prompt), prompt).first -
                          h.begin();
    const size_t keep = std::min(common, (size_t)n_prompt - 1);
    h.resize(keep);
    e->drafter.synced = std::min(e->drafter.synced, keep);
    for (size_t at = keep; at < (size_t)n_prompt; at += kChunk) {
        const int n = (int)std::min<size_t>(kChunk, (size_t)n_prompt - at);
        const bool last = at + (size_t)n == (size_t)n_prompt;
        const int rc = last ? ts5hip_forward_in_place(m, prompt + at, n, (int)at, 0)
                            : ts5hip_forward(m, prompt + at, n, (int)at, nullptr, 0);
        if (rc != TS5HIP_OK) {
            e->forget();
            return rc;
        }
        h.insert(h.end(), prompt + at, prompt + at + n);
    }
    st[S_EVAL] = (int32_t)(n_prompt - keep);

    const int full = p->draft < 0 ? 7 : std::min(p->draft, 255);  // a batch must fit one 256-row chunk
    if (full > 0) e->finder.rebuild(h);
    DraftGovernor governor(p->adapt != 0);
    int n_out = 0;
    auto emit = [&](int32_t t) {
        st[S_GEN]++;
        if (n_out < p->max_tokens) out[n_out++] = t;
    };
    auto sample_rows = [&](int nrows) { return model_pick_rows(m, 0, nrows, p->temperature, p->top_k, e->picks); };
    auto draw = [&](int row) { return model_draw(m, e->rng, e->picks, row, p->temperature, p->top_p, p->top_k); };

    if (int rc = sample_rows(1)) return rc;
    int32_t tok = draw(0);
    if (tok < 0) return tok;
    for (;;) {
        if (ends(eog, n_eog, tok)) {
            st[S_EOG] = 1;
            break;
        }
        emit(tok);
        if (st[S_GEN] >= p->max_tokens || (int)h.size() + 1 >= n_ctx) break;

        // Drafts: lookup first, the draft model where lookup finds nothing.
        std::vector<int32_t> &b = e->batch;
        b.assign(1, tok);
        const int room = std::min({governor.length(full), p->max_tokens - st[S_GEN], n_ctx - (int)h.size() - 2});
        if (room > 0) {
            const int64_t from = e->finder.find(h, tok);
            for (int64_t i = from; from >= 0 && i <= (int64_t)h.size() && (int)b.size() <= room; i++)
                b.push_back(i < (int64_t)h.size() ? h[(size_t)i] : tok);
        }
        const bool by_model = b.size() == 1 && room > 0 && e->drafter.live;
        if (by_model) e->drafter.propose(h, tok, room, model_vocab(m), eog, n_eog, b);

        // Verify: one forward of the batch, then walk its rows while the
        // target's own sample equals the next draft.
        const int nb = (int)b.size();
        const size_t pos = h.size();
        int rc = ts5hip_forward_in_place(m, b.data(), nb, (int)pos, nb > 1 ? 1 : 0);
        if (rc == TS5HIP_OK) rc = sample_rows(nb);
        if (rc != TS5HIP_OK) {
            e->forget();
            return rc;
        }
        st[S_DRAFTED] += nb - 1;
        int kept = 0;
        int32_t next = -1;
        for (int i = 0; i < nb; i++) {
            next = draw(i);
            if (next < 0) {
                e->forget();
                return next;
            }
            if (i + 1 == nb || next != b[(size_t)i + 1] || ends(eog, n_eog, next)) break;
            kept++;
        }
        st[S_ACCEPTED] += kept;
        e->by_source[by_model ? 2 : 0] += nb - 1;
        e->by_source[by_model ? 3 : 1] += kept;
        governor.judged(kept, nb - 1);
        h.insert(h.end(), b.begin(), b.begin() + kept + 1);
        if (full > 0) e->finder.extend(h);
        // The drafter forwarded the batch's tokens but its last draft.
        if (by_model && nb > 1) e->drafter.synced = std::min(h.size(), pos + (size_t)nb - 1);
        for (int i = 1; i <= kept; i++) emit(b[(size_t)i]);
        if (st[S_GEN] >= p->max_tokens) break;
        tok = next;
    }
    if (stats) std::memcpy(stats, st, sizeof st);
    return n_out;
}

}  // extern "C"
