#pragma once

// Tile-selection policies: decide which spatial tiles (or, in cross-frame
// mode, which frame-major candidates g*tiles_per_frame + t) are compacted
// into the hot KV arena for the current step. Policies are pure host code
// and never touch device memory.
//
// Interface kept from the reference (reference: src/tile_gating_policy.h:8-68):
// class names, the virtual select() signature, name() strings
// ("none", "uniform", "recency", "reuse_weighted", "motion") and the
// selection rules (reference: src/tile_gating_policy.cpp:1-83).
//
// Additive: select_range() evaluates a policy over a sub-range of the
// frame-major candidate list (used by sliding-window attention, where only
// the last W frames are attendable). select_range(s, 0, n, ...) is
// identical to select(s, n, ...). It is a non-virtual member, so the class's
// virtual table (destructor, select, name) is the reference's and a policy
// compiled against the reference header is binary compatible.

class TileGatingPolicy {
public:
    virtual ~TileGatingPolicy() {}

    // Choose up to max_tiles ids from 0..num_tiles-1 given per-candidate
    // motion scores. out_ids must hold max_tiles entries; *out_count
    // receives the number written.
    virtual void select(const float* motion_scores, int num_tiles,
                        int max_tiles, long* out_ids, int* out_count) = 0;
    virtual const char* name() const = 0;

    // Candidates are scores_flat[first_id .. first_id + num_candidates);
    // returned ids are absolute (first_id already added). Forwards to
    // select() on the shifted pointer, except for ReuseWeightedPolicy, whose
    // priorities depend on the absolute id (ReuseWeightedPolicy::select_window).
    void select_range(const float* scores_flat, long first_id,
                      int num_candidates, int max_tiles, long* out_ids,
                      int* out_count);
};

// Control: persist nothing.
class NoPersistencePolicy : public TileGatingPolicy {
public:
    void select(const float*, int, int, long*, int* out_count) override;
    const char* name() const override;
};

// Fixed leading window: ids 0..max_tiles-1 regardless of scores or count.
class UniformWindowPolicy : public TileGatingPolicy {
public:
    void select(const float*, int, int max_tiles, long* out_ids,
                int* out_count) override;
    const char* name() const override;
};

// Newest-first recency window over frame-major candidates: the last
// max_tiles candidate ids, ascending.
class RecencyWindowPolicy : public TileGatingPolicy {
public:
    void select(const float*, int num_candidates, int max_tiles,
                long* out_ids, int* out_count) override;
    const char* name() const override;
};

// priority(id) = (total_frames - id / tiles_per_frame)
//              * (1 - min(1, score / max(1e-6, max score)))
// evaluated in double; highest priority first, ties by ascending id.
class ReuseWeightedPolicy : public TileGatingPolicy {
public:
    ReuseWeightedPolicy(int tiles_per_frame, int total_frames);
    void select(const float* scores_flat, int num_candidates, int max_tiles,
                long* out_ids, int* out_count) override;
    const char* name() const override;
    // Window-aware form behind select_range: the source frame of candidate
    // i is (first_id + i) / tiles_per_frame.
    void select_window(const float* scores_flat, long first_id,
                       int num_candidates, int max_tiles, long* out_ids,
                       int* out_count);

private:
    int tpf_;
    int total_frames_;
};

// Lowest motion first (stable, so equal scores keep ascending id order).
class MotionGatedPolicy : public TileGatingPolicy {
public:
    void select(const float* motion_scores, int num_tiles, int max_tiles,
                long* out_ids, int* out_count) override;
    const char* name() const override;
};

// Factory by name ("none", "uniform", "recency", "motion", "reuse_weighted");
// returns nullptr for an unknown name. Caller owns the result (delete).
TileGatingPolicy* make_tile_gating_policy(const char* name,
                                          int tiles_per_frame,
                                          int total_frames);
