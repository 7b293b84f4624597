// The decode driver: ts5's Engine::generate (engine/src/engine.cpp:149-292)
// over this backend, with its speculation: prompt-lookup drafts
// (engine/src/engine.cpp:134-147) and, where lookup finds nothing, a draft
// model's greedy continuation (engine/src/engine.cpp:75-129), verified in one
// batched forward and kept while the target's own sample equals the draft.
//
// Host code over the library's C ABI: every forward is ts5hip_forward /
// ts5hip_forward_in_place (the batch runs on the matrix cores), every sample
// is Engine::sample on the pinned logits rows (capi.cpp sample_host_row, the
// same mt19937_64 stream). The output ids, and the counts of drafted and
// accepted tokens, are the reference's for the same model, prompt and seed.
#include <algorithm>
#include <cstring>
#include <random>
#include <string>
#include <unordered_map>
#include <vector>

#include "common_host.h"
#include "runtime.h"

using namespace ts5hip;

struct ts5hip_engine {
    ts5hip_model *m = nullptr, *dm = nullptr;
    ts5hip_sampler *rng = nullptr;  // Engine::rng_: std::mt19937_64, default-seeded
    std::vector<int32_t> cached;    // ids whose K/V the target holds, position = index
    size_t dcached = 0;             // ... and how many of them the draft model holds
    int written = 0;
    bool drafter_ok = false;
    std::unordered_map<uint64_t, int32_t> gram2, gram3;  // n-gram -> position after its last occurrence
    std::vector<int32_t> cu;
};

namespace {

uint64_t gram_key(int32_t a, int32_t b) { return ((uint64_t)(uint32_t)a << 21) | (uint32_t)b; }

// The n-grams ending at positions from.. of cached, later ones replacing
// earlier ones (a lookup finds the most recent occurrence).
void index_grams(ts5hip_engine *e, size_t from) {
    const std::vector<int32_t> &c = e->cached;
    for (size_t j = std::max<size_t>(from, 1); j < c.size(); j++) {
        e->gram2[gram_key(c[j - 1], c[j])] = (int32_t)j + 1;
        if (j >= 2) e->gram3[(gram_key(c[j - 2], c[j - 1]) << 21) | (uint32_t)c[j]] = (int32_t)j + 1;
    }
}

// Up to k drafts after `tok`: what followed the most recent earlier
// occurrence of the text's last 3-gram (then 2-gram).
void draft_lookup(ts5hip_engine *e, int32_t tok, int k, std::vector<int32_t> &out) {
    const std::vector<int32_t> &c = e->cached;
    const size_t sz = c.size();
    int32_t p = -1;
    if (sz >= 2) {
        auto it = e->gram3.find((gram_key(c[sz - 2], c[sz - 1]) << 21) | (uint32_t)tok);
        if (it != e->gram3.end()) p = it->second;
    }
    if (p < 0 && sz >= 1) {
        auto it = e->gram2.find(gram_key(c[sz - 1], tok));
        if (it != e->gram2.end()) p = it->second;
    }
    if (p < 0) return;
    for (size_t i = (size_t)p; i <= sz && (int)out.size() < k + 1; i++) out.push_back(i < sz ? c[i] : tok);
}

bool is_eog(const int32_t *eog, int n_eog, int32_t t) { return std::find(eog, eog + n_eog, t) != eog + n_eog; }

// Up to k drafts: the draft model's greedy continuation after catching its
// cache up to the confirmed history plus `tok` (a backlog of 256 or more is
// caught up one chunk per step, without drafting). A failure stops drafting
// by model, not the request.
void draft_model(ts5hip_engine *e, int32_t tok, int k, const int32_t *eog, int n_eog, std::vector<int32_t> &out) {
    ts5hip_model *dm = e->dm;
    const int nv = model_vocab(dm);
    const int pos = (int)e->cached.size();
    if (pos + k + 2 > ts5hip_n_ctx(dm)) return;
    auto fits = [&](const int32_t *p, size_t n) {
        for (size_t i = 0; i < n; i++)
            if (p[i] >= nv) {
                e->drafter_ok = false;
                return false;
            }
        return true;
    };
    const size_t CHUNK = 256;
    if (e->cached.size() - e->dcached >= CHUNK) {
        if (!fits(e->cached.data() + e->dcached, CHUNK)) return;
        if (ts5hip_forward(dm, e->cached.data() + e->dcached, (int)CHUNK, (int)e->dcached, nullptr, 0) != TS5HIP_OK) {
            e->drafter_ok = false;
            return;
        }
        e->dcached += CHUNK;
        return;
    }
    e->cu.assign(e->cached.begin() + (ptrdiff_t)e->dcached, e->cached.end());
    e->cu.push_back(tok);
    if (!fits(e->cu.data(), e->cu.size())) return;
    int32_t t = -1;
    for (int i = 0; i < k; i++) {
        const int32_t *in = i == 0 ? e->cu.data() : &t;
        const int n = i == 0 ? (int)e->cu.size() : 1;
        const int p0 = i == 0 ? (int)e->dcached : pos + i;
        if (ts5hip_forward_in_place(dm, in, n, p0, 0) != TS5HIP_OK) {
            e->drafter_ok = false;
            return;
        }
        const float *lg = ts5hip_logits_view(dm);
        t = (int32_t)(std::max_element(lg, lg + nv) - lg);
        if (t >= model_vocab(e->m)) break;  // a padded drafter row is no target token
        out.push_back(t);
        if (is_eog(eog, n_eog, t)) break;
    }
}

}  // namespace

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
    e->dm = dm;
    e->dcached = 0;
    e->drafter_ok = dm != nullptr;
    return TS5HIP_OK;
}

int ts5hip_engine_generate(ts5hip_engine *e, const int32_t *prompt, int n_prompt, const ts5hip_sample_params *p,
                           const int32_t *eog, int n_eog, int32_t *out, int32_t *stats) {
    if (!e || !prompt || !p || !out || (n_eog > 0 && !eog)) return fail(nullptr, TS5HIP_ERR_ARG, "null argument");
    ts5hip_model *m = e->m;
    ts5hip_ctx *ctx = model_ctx(m);
    if (p->seed) sampler_reseed(e->rng, p->seed);
    const int nv = model_vocab(m);
    int32_t st[6] = {n_prompt, 0, 0, 0, 0, 0};  // prompt, evaluated, generated, drafted, accepted, stopped
    if (n_prompt <= 0) return fail(ctx, TS5HIP_ERR_ARG, "empty prompt");
    if (n_prompt + 1 > ts5hip_n_ctx(m)) return fail(ctx, TS5HIP_ERR_CONTEXT_FULL, "prompt longer than the context");
    // The cached prefix is reused; the last prompt token is always evaluated.
    size_t keep = 0;
    while (keep < e->cached.size() && keep < (size_t)n_prompt && e->cached[keep] == prompt[keep]) keep++;
    if (keep == (size_t)n_prompt) keep--;
    if (keep == 0) e->written = 0;
    e->cached.resize(keep);
    if (e->dcached > keep) e->dcached = keep;
    const int chunk = 256;
    for (size_t i = keep; i < (size_t)n_prompt; i += chunk) {
        const int n = (int)std::min<size_t>(chunk, (size_t)n_prompt - i);
        const bool last = i + (size_t)n >= (size_t)n_prompt;
        const int rc = last ? ts5hip_forward_in_place(m, prompt + i, n, (int)i, 0)
                            : ts5hip_forward(m, prompt + i, n, (int)i, nullptr, 0);
        if (rc != TS5HIP_OK) {
            e->cached.clear();
            e->dcached = 0;
            return rc;
        }
        e->written = std::max(e->written, (int)(i + n));
        e->cached.insert(e->cached.end(), prompt + i, prompt + i + n);
    }
    st[1] = (int32_t)(n_prompt - keep);
    int dmax = p->draft < 0 ? 7 : std::min(p->draft, 255);
    e->gram3.clear();
    e->gram2.clear();
    if (dmax > 0) index_grams(e, 0);
    int n_out = 0;
    auto emit = [&](int32_t t) {
        st[2]++;
        if (n_out < p->max_tokens) out[n_out++] = t;
    };
    float acc = -1;  // accepted / proposed, an EWMA; < 0 until a batch has been judged
    int step = 0;
    std::vector<int32_t> batch;
    int32_t tok = sample_host_row(e->rng, ts5hip_logits_view(m), nv, p->temperature, p->top_p, p->top_k);
    while (true) {
        if (is_eog(eog, n_eog, tok)) {
            st[5] = 1;
            break;
        }
        emit(tok);
        if (st[2] >= p->max_tokens) break;
        if ((int)e->cached.size() + 1 >= ts5hip_n_ctx(m)) break;
        batch.assign(1, tok);
        int want = dmax;
        if (p->adapt && acc >= 0) {
            want = acc < 0.15f ? 0 : acc < 0.5f ? std::min(dmax, 3) : dmax;
            if (want == 0 && step % 16 == 0) want = std::min(dmax, 3);
        }
        step++;
        int room = std::min(want, p->max_tokens - st[2]);
        room = std::min(room, ts5hip_n_ctx(m) - (int)e->cached.size() - 2);
        if (room > 0) draft_lookup(e, tok, room, batch);
        const bool by_model = batch.size() == 1 && room > 0 && e->dm && e->drafter_ok;
        if (by_model) draft_model(e, tok, room, eog, n_eog, batch);
        const int nb = (int)batch.size();
        if (int rc = ts5hip_forward_in_place(m, batch.data(), nb, (int)e->cached.size(), nb > 1 ? 1 : 0)) {
            e->cached.clear();
            e->dcached = 0;
            return rc;
        }
        e->written = std::max(e->written, (int)e->cached.size() + nb);
        const float *lg = ts5hip_logits_view(m);
        st[3] += nb - 1;
        int accepted = 0;
        int32_t next = -1;
        for (int i = 0; i < nb; i++) {
            next = sample_host_row(e->rng, lg + (size_t)i * nv, nv, p->temperature, p->top_p, p->top_k);
            if (i + 1 < nb && next == batch[i + 1] && !is_eog(eog, n_eog, next)) {
                accepted++;
                continue;
            }
            break;
        }
        st[4] += accepted;
        if (nb > 1) {
            const float r = (float)accepted / (float)(nb - 1);
            acc = acc < 0 ? r : 0.8f * acc + 0.2f * r;
        }
        e->cached.insert(e->cached.end(), batch.begin(), batch.begin() + accepted + 1);
        if (dmax > 0) index_grams(e, e->cached.size() - (size_t)(accepted + 1));
        // The drafter holds batch[0..nb-2]; with everything accepted its last
        // draft was never forwarded.
        if (by_model && batch.size() > 1) e->dcached = e->cached.size() - (accepted == nb - 1 ? 1 : 0);
        for (int i = 1; i <= accepted; i++) emit(batch[i]);
        if (st[2] >= p->max_tokens) break;
        tok = next;
    }
    if (stats) std::memcpy(stats, st, sizeof st);
    return n_out;
}

}  // extern "C"
