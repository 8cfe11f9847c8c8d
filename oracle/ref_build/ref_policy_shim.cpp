// TEST INFRASTRUCTURE ONLY. C entry points over the reference's own policy
// and tile-layout code, compiled from /root/reference/src (never copied) into
// oracle/_ref/libref_policy.so by oracle/ref_build/Makefile. Used to produce
// and re-check the policy golden vectors; nothing in the product links it.
#include "tile_gating_policy.h"  // reference header (-I/root/reference/src)
#include "tile_layout.h"         // reference header

#include <cstring>

extern "C" int ref_policy_select(const char* name, int tiles_per_frame, int total_frames,
                                 const float* scores, int num_candidates, int max_tiles,
                                 long* out_ids) {
    TileGatingPolicy* p = nullptr;
    if (!strcmp(name, "none")) p = new NoPersistencePolicy();
    else if (!strcmp(name, "uniform")) p = new UniformWindowPolicy();
    else if (!strcmp(name, "recency")) p = new RecencyWindowPolicy();
    else if (!strcmp(name, "motion")) p = new MotionGatedPolicy();
    else if (!strcmp(name, "reuse_weighted")) p = new ReuseWeightedPolicy(tiles_per_frame, total_frames);
    if (!p) return -1;
    int count = 0;
    p->select(scores, num_candidates, max_tiles, out_ids, &count);
    delete p;
    return count;
}

extern "C" long ref_layout_tiles_per_frame(int tpf, int tt) { return TileLayout(tpf, tt).tiles_per_frame; }
extern "C" long ref_layout_tile_start(int tpf, int tt, long id) { return TileLayout(tpf, tt).tile_start(id); }
extern "C" int ref_layout_tile_count(int tpf, int tt, long id) { return TileLayout(tpf, tt).tile_count(id); }
