// Host-side helpers shared by capi.cpp and model.cpp.
#pragma once
#include <cmath>
#include <random>
#include <vector>

#include "common.h"
#include "runtime.h"

namespace ts5hip {

// Where rows [row0, ...) of a tensor of total_rows rows start in its HBM layout.
struct SplitDst {
    void *body;
    void *scales;  // split layouts only
};
inline SplitDst split_dst(uint32_t t, int64_t ne0, int64_t total_rows, void *base, int64_t row0) {
    const int bv = block_values(t);
    const int64_t nb = ne0 / bv;
    uint8_t *b = (uint8_t *)base;
    if (split_layout(t)) {
        const int body = t == T_Q6_K ? Q6K_BODY : Q8_BODY;
        return SplitDst{b + row0 * nb * body,
                        b + split_scale_offset(t, nb * total_rows) + row0 * nb * split_scale_bytes(t)};
    }
    return SplitDst{b + (size_t)row0 * nb * gguf_block_bytes(t), nullptr};
}

// Host GGUF bytes of nrows rows -> rows [row0, row0 + nrows) of a tensor of
// total_rows rows in HBM layout (capi.cpp).
int upload_weight(ts5hip_ctx *ctx, uint32_t t, int64_t ne0, int64_t nrows, const void *gguf, void *dst, int64_t row0,
                  int64_t total_rows);

// The RoPE angles of engine/src/cpu_backend.cpp:59-61 for every position:
// theta = pos * scale * base^(-2i/n_rot) (/ freqs[i]), then (cos, sin) as
// float pairs [n_pos][n_rot/2]. Computed on the host with the same float
// operations and libm calls as the reference's CPU path.
inline void rope_table_host(int n_rot, int n_pos, float base, float scale, const float *freqs, std::vector<float> &t) {
    const int half = n_rot / 2;
    std::vector<float> inv(half);
    for (int i = 0; i < half; i++) inv[i] = std::pow(base, -2.0f * i / n_rot);
    t.resize((size_t)n_pos * half * 2);
    for (int p = 0; p < n_pos; p++) {
        for (int i = 0; i < half; i++) {
            float theta = p * scale * inv[i];
            if (freqs) theta /= freqs[i];
            t[((size_t)p * half + i) * 2] = std::cos(theta);
            t[((size_t)p * half + i) * 2 + 1] = std::sin(theta);
        }
    }
}

// Split count of the flash decode: as many work items as fit one round of
// `slots` workgroups (its 512-thread work item holds a CU, so slots = the CU
// count); a second round costs more than longer slices (5 verify queries at
// 4300 keys: 22 us with 6 splits, 37 us with 13).
inline int attn_splits(int B, int n_head_kv, int slots) {
    const int s = slots / (B * n_head_kv);
    return s < 1 ? 1 : (s > 64 ? 64 : s);  // at most 64 (the merge's table)
}
// Key splits of the multi-query batch attention: one work item a CU over the
// KV heads (all the batch's queries in each).
inline int attn_mq_splits(int n_head_kv, int slots) {
    const int s = slots / n_head_kv;
    return s < 1 ? 1 : (s > 64 ? 64 : s);
}
inline size_t attn_partial_bytes(int B, int n_split, int H, int HKV, int HD) {
    return (size_t)B * n_split * HKV * attn_group_floats(H / HKV, HD) * sizeof(float);
}

// The draw of Engine::sample (engine/src/engine.cpp:34-45) from k candidates
// sorted by descending logit: weights exp((l - l0) / T) in double, the
// shortest prefix whose cumulative share reaches top_p, then
// std::discrete_distribution on the engine's std::mt19937_64.
inline int32_t sampler_draw(std::mt19937_64 &rng, std::vector<double> &w, const int32_t *ids, const float *lg, int k,
                            float temperature, float top_p) {
    w.resize((size_t)k);
    const double top = lg[0];
    double total = 0;
    for (int i = 0; i < k; i++) total += w[i] = std::exp((lg[i] - top) / temperature);
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
    return ids[pick(rng)];
}

// Engine::sample (engine/src/engine.cpp:16-46) over rows of the last
// forward's logits, which stay in HBM: the candidates of rows
// [row0, row0 + nrows) are picked on the GPU in one pass (greedy: the first
// maximum; top-k: the best k + 1, sorted), then model_draw makes row i's draw
// on the host, with the row itself brought over only when the candidates do
// not fix the result (ties, NaN, top-k past the GPU pick) (model.cpp).
enum { PICK_GREEDY = 0, PICK_TOPK = 1, PICK_HOST = 2 };
struct RowPicks {
    int mode = PICK_HOST, row0 = 0, nrows = 0, k = 0, kk = 0;
    std::vector<float> v;
    std::vector<int32_t> id;
};
int model_pick_rows(ts5hip_model *m, int row0, int nrows, float temperature, int top_k, RowPicks &pk);
int32_t model_draw(ts5hip_model *m, ts5hip_sampler *s, const RowPicks &pk, int i, float temperature, float top_p,
                   int top_k);

// Engine::sample over a host row of logits (capi.cpp).
int32_t sample_host_row(ts5hip_sampler *s, const float *lg, int n, float temperature, float top_p, int top_k);
// Engine::generate's rng_.seed(seed) (capi.cpp).
void sampler_reseed(ts5hip_sampler *s, uint64_t seed);
// The model's vocabulary and context handle (model.cpp), for the decode driver.
int model_vocab(const ts5hip_model *m);
ts5hip_ctx *model_ctx(const ts5hip_model *m);

}  // namespace ts5hip
