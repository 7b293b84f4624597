// TEST INFRASTRUCTURE ONLY: part of the CPU oracle (see ts5_oracle.h).
//
// Engine::sample, restated from engine/src/engine.cpp:16-46: greedy is the
// first maximum; otherwise the top k by a min-heap over the vocabulary, sorted
// by descending logit, weights exp((l - l_max) / T) in double, the shortest
// prefix whose cumulative share reaches top_p, and a
// std::discrete_distribution draw on a std::mt19937_64 (engine/src/engine.h:73).
#include <algorithm>
#include <cmath>
#include <random>
#include <vector>

#include "ts5_oracle.h"

struct ts5o_sampler {
    std::mt19937_64 rng;
    std::vector<int32_t> heap;
};

namespace {

int32_t draw(ts5o_sampler *s, const float *lg, const int32_t *order, int k, float temperature, float top_p) {
    std::vector<double> w((size_t)k);
    const double top = lg[order[0]];
    double total = 0;
    for (int i = 0; i < k; i++) total += w[i] = std::exp((lg[order[i]] - top) / temperature);
    double run = 0;
    int keep = k;
    for (int i = 0; i < k; i++) {
        run += w[i] / total;
        if (run >= top_p) {
            keep = i + 1;
            break;
        }
    }
    std::discrete_distribution<int> pick(w.begin(), w.begin() + keep);
    return order[pick(s->rng)];
}

}  // namespace

extern "C" {

ts5o_sampler *ts5o_sampler_new(uint64_t seed) {
    ts5o_sampler *s = new ts5o_sampler();
    s->rng.seed(seed);
    return s;
}

void ts5o_sampler_free(ts5o_sampler *s) { delete s; }

int32_t ts5o_sample(ts5o_sampler *s, const float *lg, int n, float temperature, float top_p, int top_k) {
    if (temperature <= 0) return (int32_t)(std::max_element(lg, lg + n) - lg);
    const int k = top_k > 0 ? std::min(top_k, n) : n;
    // The heap's front is the smallest logit kept so far.
    auto above = [lg](int32_t a, int32_t b) { return lg[a] > lg[b]; };
    std::vector<int32_t> &h = s->heap;
    h.clear();
    for (int32_t i = 0; i < n; i++) {
        if ((int)h.size() < k) {
            h.push_back(i);
            std::push_heap(h.begin(), h.end(), above);
        } else if (lg[i] > lg[h.front()]) {
            std::pop_heap(h.begin(), h.end(), above);
            h.back() = i;
            std::push_heap(h.begin(), h.end(), above);
        }
    }
    std::sort_heap(h.begin(), h.end(), above);
    return draw(s, lg, h.data(), k, temperature, top_p);
}

int32_t ts5o_sample_topk(ts5o_sampler *s, const int32_t *ids, const float *logits, int k, float temperature,
                         float top_p) {
    // Candidates arrive as (id, logit) pairs already in order.
    std::vector<int32_t> order((size_t)k);
    for (int i = 0; i < k; i++) order[i] = i;
    const int32_t local = draw(s, logits, order.data(), k, temperature, top_p);
    return ids[local];
}

}  // extern "C"
