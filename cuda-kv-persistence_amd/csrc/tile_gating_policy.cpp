// Tile gating policies (host C++). Selection rules follow the reference
// (reference: src/tile_gating_policy.cpp:1-83); they must, because the
// selected ids decide the arena contents and KVMap, which are compared
// bit-exactly against the reference's behaviour.

#include "tile_gating_policy.h"

#include <algorithm>
#include <cstring>
#include <numeric>
#include <vector>

void TileGatingPolicy::select_range(const float* scores_flat, long first_id,
                                    int num_candidates, int max_tiles,
                                    long* out_ids, int* out_count) {
    if (ReuseWeightedPolicy* rw = dynamic_cast<ReuseWeightedPolicy*>(this)) {
        rw->select_window(scores_flat, first_id, num_candidates, max_tiles, out_ids, out_count);
        return;
    }
    select(scores_flat ? scores_flat + first_id : nullptr, num_candidates,
           max_tiles, out_ids, out_count);
    for (int i = 0; i < *out_count; ++i) out_ids[i] += first_id;
}

// none: never selects (reference: tile_gating_policy.cpp:6-11).
void NoPersistencePolicy::select(const float*, int, int, long*, int* out_count) {
    *out_count = 0;
}
const char* NoPersistencePolicy::name() const { return "none"; }

// uniform: the leading max_tiles ids, independent of the candidate count
// (reference: tile_gating_policy.cpp:13-19).
void UniformWindowPolicy::select(const float*, int, int max_tiles, long* out_ids,
                                 int* out_count) {
    const int n = max_tiles > 0 ? max_tiles : 0;
    for (int i = 0; i < n; ++i) out_ids[i] = i;
    *out_count = n;
}
const char* UniformWindowPolicy::name() const { return "uniform"; }

// recency: the newest max_tiles candidates in ascending order
// (reference: tile_gating_policy.cpp:21-30).
void RecencyWindowPolicy::select(const float*, int num_candidates, int max_tiles,
                                 long* out_ids, int* out_count) {
    const int first = std::max(0, num_candidates - std::max(0, max_tiles));
    int n = 0;
    for (int id = first; id < num_candidates; ++id) out_ids[n++] = id;
    *out_count = n;
}
const char* RecencyWindowPolicy::name() const { return "recency"; }

ReuseWeightedPolicy::ReuseWeightedPolicy(int tiles_per_frame, int total_frames)
    : tpf_(tiles_per_frame > 0 ? tiles_per_frame : 1), total_frames_(total_frames) {}

void ReuseWeightedPolicy::select(const float* scores_flat, int num_candidates,
                                 int max_tiles, long* out_ids, int* out_count) {
    select_window(scores_flat, 0, num_candidates, max_tiles, out_ids, out_count);
}

// reuse_weighted (reference: tile_gating_policy.cpp:32-68):
//   rate_max = max(1e-6f, max score)            (float)
//   prio(i)  = (total_frames - src_frame(i)) * (1 - min(1, s_i / rate_max))
// computed in double; sort by prio descending, then id ascending.
void ReuseWeightedPolicy::select_window(const float* scores_flat, long first_id,
                                        int num_candidates, int max_tiles,
                                        long* out_ids, int* out_count) {
    const int n = std::max(0, num_candidates);
    const float* s = scores_flat + first_id;
    float rate_max = 1e-6f;
    for (int i = 0; i < n; ++i) rate_max = std::max(rate_max, s[i]);
    const double rate_max_d = static_cast<double>(rate_max);

    std::vector<double> prio(n);
    for (int i = 0; i < n; ++i) {
        const long id = first_id + i;
        const double remaining = static_cast<double>(total_frames_ - id / tpf_);
        const double rate = std::min(1.0, static_cast<double>(s[i]) / rate_max_d);
        prio[i] = remaining * (1.0 - rate);
    }
    std::vector<int> order(n);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
        if (prio[a] != prio[b]) return prio[a] > prio[b];
        return a < b;
    });
    const int take = std::min(n, std::max(0, max_tiles));
    for (int i = 0; i < take; ++i) out_ids[i] = first_id + order[i];
    *out_count = take;
}
const char* ReuseWeightedPolicy::name() const { return "reuse_weighted"; }

// motion: ascending score, stable so ties keep id order
// (reference: tile_gating_policy.cpp:70-83).
void MotionGatedPolicy::select(const float* motion_scores, int num_tiles,
                               int max_tiles, long* out_ids, int* out_count) {
    const int n = std::max(0, num_tiles);
    std::vector<int> order(n);
    std::iota(order.begin(), order.end(), 0);
    std::stable_sort(order.begin(), order.end(), [&](int a, int b) {
        return motion_scores[a] < motion_scores[b];
    });
    const int take = std::min(n, std::max(0, max_tiles));
    for (int i = 0; i < take; ++i) out_ids[i] = order[i];
    *out_count = take;
}
const char* MotionGatedPolicy::name() const { return "motion"; }

TileGatingPolicy* make_tile_gating_policy(const char* name, int tiles_per_frame,
                                          int total_frames) {
    if (!name) return nullptr;
    if (!strcmp(name, "none")) return new NoPersistencePolicy();
    if (!strcmp(name, "uniform")) return new UniformWindowPolicy();
    if (!strcmp(name, "recency")) return new RecencyWindowPolicy();
    if (!strcmp(name, "motion")) return new MotionGatedPolicy();
    if (!strcmp(name, "reuse_weighted"))
        return new ReuseWeightedPolicy(tiles_per_frame, total_frames);
    return nullptr;
}
