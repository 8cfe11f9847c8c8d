// Frame pipeline: the reference driver's per-frame loop
// (reference: src/run_policy_experiment.cu:136-283) as a reusable library
// object behind kvp_pipeline_*.
//
// Per frame f (policies other than "none"):
//   1. policy select over the frame's tiles (intra) or the frame-major
//      candidate prefix (cross), or only the window's frames when a sliding
//      window is set;
//   2. streaming: release the rows of tiles that dropped out of the
//      selection, before staging (gid ascending, rows ascending);
//   3. arena_begin_step, KVMap prefix [0, (f+1)*T) reset to -1, then every
//      selected tile's rows staged in policy order, rows ascending, the map
//      entry of each staged row set to its arena row / slot;
//   4. the row copies and the KVMap entries that change, as one launch;
//   5. attention for the frame.
//
// Two ways to run it:
//   * kvp_pipeline_step(f): frame by frame on one arena, exactly the
//     reference's sequence; a host mirror of the device KVMap gives the exact
//     difference to the map the reference driver would upload for the frame
//     (prefix reset to -1, then the staged rows).
//   * kvp_pipeline_run: a whole layer in two launches. Steps 1-3 run on the
//     host for every frame first (a bookkeeping-only manager takes the same
//     decisions: which rows each frame maps); then one staging launch and one
//     attention launch cover every frame. K and V are fixed for the whole
//     layer, so a row holds the same bytes in every frame that maps it. The
//     layer arena gives each tile that some frame maps physical rows for the
//     longest prefix of it that any frame maps, whole tiles in key order, and
//     frame f's slice of the layer map points each of its mapped rows at
//     that row's physical row. The staging launch copies those tile prefixes
//     (as runs of consecutive rows), writes the map entries that differ from
//     the previous run (as runs) and, in bf16, the changed group-descriptor
//     entries of every slice. The arena is allocated once, at frames x the
//     rows of the set-aside (no frame maps more), and never grows; a plan past
//     it is an error. Every frame maps exactly the rows the single arena maps
//     at that frame, holding the same bytes: outputs are bitwise equal across
//     policies and modes within kvp_pipeline_run, and equal stepping's up to
//     the rounding of stepping's key split (the layer launch never splits).
//     A failure after the layer state was touched tears it down, and the
//     next run rebuilds it from scratch.
// Nothing synchronises the host per frame; all device work is ordered on the
// pipeline's stream.

#include <algorithm>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

#include "group_desc.h"
#include "kv_tile_manager.h"
#include "kvp_c_api.h"
#include "kvp_internal.h"
#include "tile_gating_policy.h"

namespace {

struct Pipeline {
    std::unique_ptr<TileGatingPolicy> policy;
    bool persist = false;
    bool cross = false;
    bool streaming = false;
    bool plan_only = false;
    int frames = 0, T = 0, D = 0, heads = 0, tile_tokens = 0, window = 0, dtype = 0;
    int elem = 4;
    long num_tiles = 0;
    long slots = 0;
    long set_aside = 0;
    std::unique_ptr<KVTileManager> mgr;
    std::vector<long> h_map;
    long* d_map = nullptr;
    std::vector<long> ids;
    int count = 0;
    std::vector<char> selected, prev_selected;
    std::vector<long> map_rows, map_slots;   // entries of this step
    std::vector<long> dev_mirror;            // current device map content
    std::vector<long> dev_rows;              // rows with a non-negative entry
    std::vector<int> stamp;                  // step id that mapped a row
    int step_id = 0;
    std::vector<long> upd_rows, upd_vals;    // entries sent to the device
    long staged_tiles = 0;
    long copy_rows = 0;
    int next_frame = 0;
    void* stream = nullptr;
    bool cold_rows_nt = false;

    // layer mode (kvp_pipeline_run)
    std::unique_ptr<KVTileManager> layer_mgr;  // bookkeeping only
    char* layer_arena = nullptr;               // layer_cap physical rows
    long region_rows = 0;                      // rows one frame may map
    long layer_cap = 0;                        // physical rows of the layer arena
    long* layer_map = nullptr;                 // frames slices of map_stride entries
    long map_stride = 0;
    long seg_space = 0;                        // tiles one map slice can hold
    // A frame's mapped rows, a tile at a time: rows [0, n) of tile gsrc
    // (frame-major tile id over all frames), at map slice index idx.
    struct Seg {
        long idx;
        long gsrc;
        int n;
    };
    std::vector<std::vector<Seg>> frame_segs;  // per frame: its segments this run
    std::vector<std::vector<int>> seg_n;       // per frame: rows mapped per tile on the device
    std::vector<std::vector<long>> seg_phys;   // per frame: their first physical row
    std::vector<std::vector<long>> seg_list;   // per frame: tiles with seg_n > 0
    std::vector<int> seg_mark;                 // tile idx -> frame plan that maps it
    int seg_gen = 0;
    std::vector<long> tile_phys;               // gsrc -> first physical row this run
    std::vector<int> tile_gen;                 // run that last mapped the tile
    std::vector<int> tile_rows;                // gsrc -> longest prefix any frame maps
    int layer_gen = 0;
    // group descriptors of the layer map (bf16): frames tables of gd_stride
    // entries; per frame, the non-empty entries the device holds
    unsigned* layer_gd = nullptr;
    long gd_stride = 0;
    std::vector<std::vector<kvp::gd::Ent>> gd_dev;
    std::vector<kvp::gd::Sub> gd_subs;
    std::vector<kvp::gd::Ent> gd_new;
    std::vector<kvp::LayerGdWrite> gd_writes;
    std::vector<unsigned> plan_gd;             // plan-only: the tables on the host
    long layer_nphys = 0;                      // physical rows assigned this run
    std::vector<long> tile_slots;              // slots of one tile (host map)
    std::vector<kvp::LayerCopyRun> layer_copies;
    std::vector<kvp::LayerMapRun> layer_updates;
    void* layer_stager = nullptr;
    KVTileManager* last_mgr = nullptr;         // manager of the last step or run
    // plan-only layer runs: the staging launch applied on the host
    std::vector<long> plan_map;                // the layer map
    std::vector<long> plan_src;                // physical row -> K/V row
    std::vector<int> plan_stamp;               // run that wrote a map entry

    ~Pipeline() {
        mgr.reset();
        layer_mgr.reset();
        if (d_map || layer_arena || layer_map || layer_stager) kvp_stream_sync(stream);
        if (layer_stager) kvp_stager_destroy(layer_stager);
        if (d_map) kvp_dev_free(d_map);
        if (layer_arena) kvp_dev_free(layer_arena);
        if (layer_map) kvp_dev_free(layer_map);
        if (layer_gd) kvp_dev_free(layer_gd);
    }
};

Pipeline* PL(void* p) { return static_cast<Pipeline*>(p); }

long window_first_frame(const Pipeline& p, int f) {
    return (p.cross && p.window > 0 && f + 1 > p.window) ? f + 1 - p.window : 0;
}

// Steps 1-2 of a gated frame on manager `mgr`: selection (ids in p.ids,
// p.count of them) and the streaming release of tiles that dropped out.
int select_and_release(Pipeline& p, KVTileManager& mgr, int f, const float* scores_flat) {
    const long T = p.T;
    if (!scores_flat) {
        kvp::set_error("pipeline: policy %s needs motion scores", p.policy->name());
        return 1;
    }
    const long kb_frame = window_first_frame(p, f);

    if (f == 0) {
        p.prev_selected.clear();
        if (p.streaming && !mgr.streaming_begin()) {
            kvp::set_error("pipeline: streaming_begin failed");
            return 1;
        }
    }

    // 1. selection
    p.count = 0;
    if (p.cross) {
        const long first = kb_frame * p.num_tiles;
        const long n = (long)(f + 1) * p.num_tiles - first;
        p.policy->select_range(scores_flat, first, (int)n, (int)p.slots, p.ids.data(), &p.count);
    } else {
        p.policy->select(scores_flat + (long)f * p.num_tiles, (int)p.num_tiles, (int)p.slots,
                         p.ids.data(), &p.count);
    }

    // 2. streaming release of tiles that dropped out
    p.selected.assign((size_t)((f + 1) * p.num_tiles), 0);
    for (int i = 0; i < p.count; ++i) {
        const long id = p.ids[i];
        if (id >= 0 && id < (long)p.selected.size()) p.selected[(size_t)id] = 1;
    }
    if (p.streaming && f > 0) {
        const long prev_len = (long)p.prev_selected.size();
        for (long gid = 0; gid < prev_len; ++gid) {
            if (!p.prev_selected[(size_t)gid]) continue;
            if (gid < (long)p.selected.size() && p.selected[(size_t)gid]) continue;
            // Intra mode releases rows of the CURRENT frame, as the
            // reference driver does (src/run_policy_experiment.cu:180-185).
            const long src_f = p.cross ? gid / p.num_tiles : f;
            const long tile = p.cross ? gid % p.num_tiles : gid;
            const long t0 = tile * p.tile_tokens;
            const long c = std::min((long)p.tile_tokens, T - t0);
            for (long r = 0; r < c; ++r) mgr.streaming_release(src_f * T + t0 + r);
        }
    }
    return 0;
}

// Steps 1-3 of a gated frame on manager `mgr`: selection, streaming release
// and staging, leaving the frame's mapped rows in p.map_rows / p.map_slots
// and its host map in p.h_map. Host bookkeeping only (a manager with a device
// arena records its copies for the next flush).
int plan_frame_host(Pipeline& p, KVTileManager& mgr, int f, const char* k, const char* v,
                    const float* scores_flat) {
    const long T = p.T;
    const long row_bytes = (long)p.D * p.elem;
    if (select_and_release(p, mgr, f, scores_flat)) return 1;

    // 3. staging + host map
    mgr.arena_begin_step();
    std::fill(p.h_map.begin(), p.h_map.begin() + (size_t)(f + 1) * T, -1L);
    p.map_rows.clear();
    p.map_slots.clear();
    p.staged_tiles = 0;
    p.copy_rows = 0;
    for (int i = 0; i < p.count; ++i) {
        const long gid = p.ids[i];
        const long src_f = p.cross ? gid / p.num_tiles : f;
        const long tile = p.cross ? gid % p.num_tiles : gid;
        // uniform hands out ids 0..slots-1 whatever the candidate count; an
        // id past the last frame names rows outside K/V and stages nothing
        // (the reference would read past its buffers)
        if (src_f >= p.frames) continue;
        const long t0 = tile * p.tile_tokens;
        const long c = std::min((long)p.tile_tokens, T - t0);
        bool all = true;
        for (long r = 0; r < c && all; ++r) {
            const long row_id = src_f * T + t0 + r;
            const char* kp = k ? k + row_id * row_bytes : nullptr;
            const char* vp = v ? v + row_id * row_bytes : nullptr;
            long slot = -1;
            if (p.streaming) {
                bool restaged = false;
                all = mgr.streaming_stage(row_id, kp, (size_t)row_bytes, vp, (size_t)row_bytes,
                                          false, &slot, &restaged);
                if (all && restaged) ++p.copy_rows;
            } else {
                all = mgr.arena_stage(kp, (size_t)row_bytes, vp, (size_t)row_bytes, &slot);
                if (all) ++p.copy_rows;
            }
            if (all) {
                p.h_map[(size_t)row_id] = slot;
                p.map_rows.push_back(row_id);
                p.map_slots.push_back(slot);
            }
        }
        if (all) ++p.staged_tiles;
    }
    return 0;
}

// Steps 1-4 of a gated frame in step mode: the host plan, then the row copies
// and changed map entries prepared as one staging plan (*plan; launched by
// the caller, not here).
int plan_frame(Pipeline& p, int f, const char* k, const char* v, const float* scores_flat,
               void** plan) {
    *plan = nullptr;
    KVTileManager& mgr = *p.mgr;
    p.last_mgr = &mgr;
    if (plan_frame_host(p, mgr, f, k, v, scores_flat)) return 1;

    // 4. row copies + changed map entries, as one staging plan
    if (!p.plan_only) {
        ++p.step_id;
        p.upd_rows.clear();
        p.upd_vals.clear();
        for (size_t i = 0; i < p.map_rows.size(); ++i) {
            const long r = p.map_rows[i];
            p.stamp[(size_t)r] = p.step_id;
            if (p.dev_mirror[(size_t)r] != p.map_slots[i]) {
                p.upd_rows.push_back(r);
                p.upd_vals.push_back(p.map_slots[i]);
                p.dev_mirror[(size_t)r] = p.map_slots[i];
            }
        }
        for (long r : p.dev_rows) {
            if (p.stamp[(size_t)r] != p.step_id && p.dev_mirror[(size_t)r] != -1) {
                p.upd_rows.push_back(r);
                p.upd_vals.push_back(-1);
                p.dev_mirror[(size_t)r] = -1;
            }
        }
        p.dev_rows = p.map_rows;
        if (!mgr.flush_plan(plan, p.d_map, 0, p.upd_rows.data(), p.upd_vals.data(),
                            p.upd_rows.size())) {
            return 1;
        }
    }
    if (p.streaming)
        (void)mgr.streaming_apply_window();
    else
        (void)mgr.arena_apply_window();
    return 0;
}

// Step 5: the frame's attention launch.
int launch_frame(Pipeline& p, int f, const char* q, const char* k, const char* v, char* out) {
    const long T = p.T;
    const long frame_bytes = T * (long)p.D * p.elem;
    kvp::AttnLaunch L;
    L.dtype = p.dtype;
    L.q = q + f * frame_bytes;
    L.out = out + f * frame_bytes;
    L.arena = p.persist ? p.mgr->arena_device_ptr() : nullptr;
    L.kvmap = p.persist ? p.d_map : nullptr;
    L.nq = p.T;
    L.D = p.D;
    L.heads = p.heads;
    L.cold_rows_nt = p.cold_rows_nt;
    L.stream = p.stream;
    if (p.cross) {
        L.k = k;
        L.v = v;
        L.key_begin = window_first_frame(p, f) * T;
        L.key_end = (long)(f + 1) * T;
    } else {
        L.k = k + f * frame_bytes;
        L.v = v + f * frame_bytes;
        if (L.kvmap) L.kvmap += (long)f * T;
        L.key_begin = 0;
        L.key_end = T;
    }
    return kvp::launch_attention(L);
}

// Step 6: end of the frame's step in the manager.
void finish_frame(Pipeline& p, KVTileManager& mgr, int f) {
    if (p.streaming)
        p.prev_selected = p.selected;
    else
        mgr.arena_end_step();
    if (p.streaming && f + 1 == p.frames) mgr.streaming_end();
}

bool check_data(const Pipeline& p, const char* q, const char* k, const char* v, const char* out) {
    if (!p.plan_only && (!q || !k || !v || !out)) {
        kvp::set_error("pipeline: null q/k/v/out");
        return false;
    }
    return true;
}

// One frame, in order: plan, staging launch, attention launch, step end.
int step_frame(Pipeline& p, int f, const char* q, const char* k, const char* v, char* out,
               const float* scores_flat) {
    if (f != p.next_frame) {
        kvp::set_error("pipeline: frame %d stepped out of order (expected %d)", f, p.next_frame);
        return 1;
    }
    if (!check_data(p, q, k, v, out)) return 1;
    if (!p.persist) {
        p.count = 0;
        p.staged_tiles = 0;
        p.copy_rows = 0;
        p.next_frame = (f + 1 == p.frames) ? 0 : f + 1;
        if (p.plan_only) return 0;
        return launch_frame(p, f, q, k, v, out);
    }
    void* plan = nullptr;
    int rc = plan_frame(p, f, k, v, scores_flat, &plan);
    if (rc == 0 && plan) rc = kvp::stage_plan_launch(plan, p.stream);
    kvp::stage_plan_free(plan);
    if (rc == 0 && !p.plan_only) rc = launch_frame(p, f, q, k, v, out);
    if (rc) return rc;
    finish_frame(p, *p.mgr, f);
    p.next_frame = (f + 1 == p.frames) ? 0 : f + 1;
    return 0;
}

// Key range [b, e) of frame f in the layer launch, in key-index space (the
// absolute key rows in cross mode, frame-relative rows in intra mode).
void frame_range(const Pipeline& p, int f, long& b, long& e) {
    if (p.cross) {
        e = (long)(f + 1) * p.T;
        b = window_first_frame(p, f) * p.T;
    } else {
        b = 0;
        e = p.T;
    }
}

// Frees the layer-mode state (device buffers after draining the stream, the
// bookkeeping manager and every host mirror of device content). The next
// run builds it again from scratch: after a failed run the device map and
// descriptor tables may not match their host mirrors any more.
void layer_teardown(Pipeline& p) {
    if (p.layer_arena || p.layer_map || p.layer_gd || p.layer_stager) (void)kvp_stream_sync(p.stream);
    if (p.layer_stager) kvp_stager_destroy(p.layer_stager);
    if (p.layer_arena) kvp_dev_free(p.layer_arena);
    if (p.layer_map) kvp_dev_free(p.layer_map);
    if (p.layer_gd) kvp_dev_free(p.layer_gd);
    p.layer_stager = nullptr;
    p.layer_arena = nullptr;
    p.layer_map = nullptr;
    p.layer_gd = nullptr;
    p.layer_mgr.reset();
    if (p.last_mgr != p.mgr.get()) p.last_mgr = nullptr;
    p.layer_cap = 0;
    p.layer_nphys = 0;
    p.gd_stride = 0;
    p.frame_segs.clear();
    p.seg_n.clear();
    p.seg_phys.clear();
    p.seg_list.clear();
    p.seg_mark.clear();
    p.tile_phys.clear();
    p.tile_gen.clear();
    p.tile_rows.clear();
    p.gd_dev.clear();
    p.plan_map.clear();
    p.plan_stamp.clear();
    p.plan_gd.clear();
}

// Layer-mode state, created at the first kvp_pipeline_run (and again after
// a failed run): the bookkeeping manager and tile tables, and (unless
// plan-only) the device arena, map, descriptor tables and stager. All or
// nothing: on any failure everything created here is released again.
int layer_setup(Pipeline& p) {
    if (p.layer_mgr) return 0;
    const long row_bytes = (long)p.D * p.elem;
    const size_t stride_floats = (size_t)2 * row_bytes / sizeof(float);
    p.layer_mgr.reset(new (std::nothrow) KVTileManager((size_t)p.set_aside, (size_t)p.set_aside));
    if (!p.layer_mgr || !p.layer_mgr->init() ||
        !p.layer_mgr->arena_attach(nullptr, (size_t)p.set_aside, stride_floats)) {
        layer_teardown(p);
        kvp::set_error("pipeline: layer manager init failed");
        return 1;
    }
    // A frame maps at most region_rows rows (the budget / slot capacity), as
    // a prefix of each tile it maps. The layer arena gives every tile the
    // longest prefix any frame of the layer maps, so it never holds more
    // than frames * region_rows rows: the reference's per-step arena summed
    // over the layer's frames (frames * set_aside bytes).
    p.region_rows = p.set_aside / (2 * row_bytes);
    p.layer_cap = std::min((long)p.frames * p.region_rows, (long)p.frames * p.T);
    p.map_stride = p.cross ? (long)p.frames * p.T : (long)p.T;
    p.seg_space = p.cross ? (long)p.frames * p.num_tiles : p.num_tiles;
    const long map_entries = (long)p.frames * p.map_stride;
    long span = p.T;
    if (p.cross) span = (long)(p.window > 0 ? std::min(p.window, p.frames) : p.frames) * p.T;
    // descriptors serve the bf16 kernel only
    p.gd_stride = p.dtype == 1 ? 4 * ((span + 63) / 64) : 0;
    const long gd_entries = (long)p.frames * p.gd_stride;
    p.frame_segs.assign((size_t)p.frames, {});
    p.seg_n.assign((size_t)p.frames, std::vector<int>((size_t)p.seg_space, 0));
    p.seg_phys.assign((size_t)p.frames, std::vector<long>((size_t)p.seg_space, -1L));
    p.seg_list.assign((size_t)p.frames, {});
    p.seg_mark.assign((size_t)p.seg_space, 0);
    p.tile_phys.assign((size_t)p.frames * p.num_tiles, -1L);
    p.tile_gen.assign((size_t)p.frames * p.num_tiles, 0);
    p.tile_rows.assign((size_t)p.frames * p.num_tiles, 0);
    p.tile_slots.assign((size_t)p.tile_tokens, -1L);
    p.gd_dev.assign((size_t)p.frames, {});
    if (p.plan_only) {
        p.plan_map.assign((size_t)map_entries, -1L);
        p.plan_stamp.assign((size_t)map_entries, 0);
        p.plan_gd.assign((size_t)gd_entries * 2, 0u);
        return 0;
    }
    p.layer_arena = static_cast<char*>(
        kvp_dev_alloc((size_t)std::max<long>(1, p.layer_cap * 2 * row_bytes)));
    p.layer_map = static_cast<long*>(kvp_dev_alloc((size_t)map_entries * sizeof(long)));
    if (gd_entries > 0)
        p.layer_gd = static_cast<unsigned*>(kvp_dev_alloc((size_t)gd_entries * 8));
    p.layer_stager = kvp_stager_create();
    if (!p.layer_arena || !p.layer_map || (gd_entries > 0 && !p.layer_gd) || !p.layer_stager) {
        layer_teardown(p);
        kvp::set_error("pipeline: layer arena / map allocation failed");
        return 1;
    }
    // the device map starts as all -1 (matching seg_n), the descriptor
    // tables as all "no arena row" (matching gd_dev)
    if (kvp_stage_run(p.layer_stager, nullptr, 0, nullptr, 0, p.layer_map, map_entries, nullptr,
                      nullptr, 0, p.stream) ||
        kvp::fill_words(p.layer_gd, gd_entries * 2, 0u, p.stream)) {
        const std::string err = kvp_last_error();
        layer_teardown(p);
        kvp::set_error("%s", err.c_str());
        return 1;
    }
    return 0;
}

// Step 3 of a gated frame in layer mode, a tile at a time: the manager
// takes the decisions of plan_frame_host's row loop (batched per tile, same
// order, same stop at a tile's first refused row), and the frame's mapped
// rows are kept as segments in p.frame_segs[f] (and their tiles marked as
// mapped this run, with the longest prefix mapped). The host map is written
// for the last frame of the layer only (introspection of the last step).
void plan_frame_layer(Pipeline& p, KVTileManager& mgr, int f, const char* k, const char* v) {
    const long T = p.T;
    const long row_bytes = (long)p.D * p.elem;
    const bool last = f + 1 == p.frames;
    mgr.arena_begin_step();
    if (last) std::fill(p.h_map.begin(), p.h_map.begin() + (size_t)(f + 1) * T, -1L);
    std::vector<Pipeline::Seg>& segs = p.frame_segs[(size_t)f];
    segs.clear();
    p.staged_tiles = 0;
    p.copy_rows = 0;
    for (int i = 0; i < p.count; ++i) {
        const long gid = p.ids[i];
        const long src_f = p.cross ? gid / p.num_tiles : f;
        const long tile = p.cross ? gid % p.num_tiles : gid;
        // uniform hands out ids 0..slots-1 whatever the candidate count; an
        // id past the last frame names rows outside K/V and stages nothing
        if (src_f >= p.frames) continue;
        const long t0 = tile * p.tile_tokens;
        const long c = std::min((long)p.tile_tokens, T - t0);
        const long row0 = src_f * T + t0;
        const char* kp = k ? k + row0 * row_bytes : nullptr;
        const char* vp = v ? v + row0 * row_bytes : nullptr;
        long* slots = last ? p.tile_slots.data() : nullptr;
        long n, copied = 0;
        if (p.streaming) {
            n = mgr.streaming_stage_rows(row0, kp, (size_t)row_bytes, vp, (size_t)row_bytes, c,
                                         slots, &copied);
        } else {
            n = mgr.arena_stage_rows(kp, (size_t)row_bytes, vp, (size_t)row_bytes, c, slots);
            copied = n;
        }
        p.copy_rows += copied;
        if (last)
            for (long j = 0; j < n; ++j) p.h_map[(size_t)(row0 + j)] = p.tile_slots[(size_t)j];
        if (n == c) ++p.staged_tiles;
        if (n > 0) {
            const long gsrc = src_f * p.num_tiles + tile;
            segs.push_back(Pipeline::Seg{p.cross ? gsrc : tile, gsrc, (int)n});
            if (p.tile_gen[(size_t)gsrc] != p.layer_gen) {
                p.tile_gen[(size_t)gsrc] = p.layer_gen;
                p.tile_rows[(size_t)gsrc] = 0;
            }
            p.tile_rows[(size_t)gsrc] = std::max(p.tile_rows[(size_t)gsrc], (int)n);
        }
    }
}

// Copy of c K/V rows from row `row` to physical rows [phys, phys + c),
// appended to the run table: runs of consecutive rows (also across tiles)
// of at most ~12 KiB each, which one workgroup of the staging kernel moves
// in a single pass of loads (one round trip to memory per run).
void layer_add_copy(Pipeline& p, long row, long phys, long c) {
    const long row_bytes = 2L * p.D * p.elem;
    const long per_run = std::max<long>(1, std::min<long>(kvp::kLayerCopyRows, 12288 / row_bytes));
    while (c > 0) {
        if (!p.layer_copies.empty()) {
            kvp::LayerCopyRun& r = p.layer_copies.back();
            if (r.n < per_run && r.src_row + r.n == row && r.dst_row + r.n == phys) {
                const long k = std::min(c, per_run - r.n);
                r.n += (int)k;
                row += k;
                phys += k;
                c -= k;
                continue;
            }
        }
        const long k = std::min(c, per_run);
        p.layer_copies.push_back(kvp::LayerCopyRun{(int)row, (int)phys, (int)k, 0});
        row += k;
        phys += k;
        c -= k;
    }
}

// Map entries [index, index + n) set to value + j (value -1: reset).
void layer_add_update(Pipeline& p, long index, long value, long n) {
    for (long j = 0; j < n; j += kvp::kLayerMapEntries)
        p.layer_updates.push_back(kvp::LayerMapRun{
            index + j, value < 0 ? -1 : (int)(value + j),
            (int)std::min<long>(kvp::kLayerMapEntries, n - j)});
}

// Physical rows of the run: every tile some frame maps, its longest mapped
// prefix, in key order (tile id order is key-row order, across frames too),
// so the arena rows of adjacent mapped tiles are adjacent and a 16-row copy
// group of the attention kernel whose rows are all mapped is one run of
// arena rows. One copy run table for all of them.
int layer_assign(Pipeline& p) {
    const long T = p.T;
    const long ntiles = (long)p.frames * p.num_tiles;
    for (long g = 0; g < ntiles; ++g) {
        if (p.tile_gen[(size_t)g] != p.layer_gen) continue;
        const long tile = g % p.num_tiles;
        const long row0 = (g / p.num_tiles) * T + tile * p.tile_tokens;
        const long c = p.tile_rows[(size_t)g];
        if (p.layer_nphys + c > p.layer_cap || row0 + c > 0x7fffffffL) {
            kvp::set_error("pipeline: the layer maps more than its %ld arena rows", p.layer_cap);
            return 1;
        }
        p.tile_phys[(size_t)g] = p.layer_nphys;
        layer_add_copy(p, row0, p.layer_nphys, c);
        p.layer_nphys += c;
    }
    return 0;
}

// Frame f's map runs: the entries of map slice f that differ from what the
// device holds. Write runs cover the rows a tile maps now; reset runs only
// rows no tile of the frame maps now, so the runs of one launch never
// overlap.
void layer_collect(Pipeline& p, int f) {
    const long T = p.T;
    const long base = (long)f * p.map_stride;
    const long rel = p.cross ? 0 : (long)f * T;  // intra slices are frame-relative
    std::vector<int>& sn = p.seg_n[(size_t)f];
    std::vector<long>& sp = p.seg_phys[(size_t)f];
    std::vector<long>& list = p.seg_list[(size_t)f];
    const std::vector<Pipeline::Seg>& segs = p.frame_segs[(size_t)f];
    ++p.seg_gen;
    for (const Pipeline::Seg& s : segs) {
        const long tile = s.gsrc % p.num_tiles;
        const long row0 = (s.gsrc / p.num_tiles) * T + tile * p.tile_tokens;
        const long ph = p.tile_phys[(size_t)s.gsrc];
        const long e0 = base + row0 - rel;
        const int old_n = sn[(size_t)s.idx];
        if (old_n != s.n || sp[(size_t)s.idx] != ph) layer_add_update(p, e0, ph, s.n);
        if (old_n > s.n) layer_add_update(p, e0 + s.n, -1, old_n - s.n);
        p.seg_mark[(size_t)s.idx] = p.seg_gen;
    }
    for (long idx : list) {
        if (p.seg_mark[(size_t)idx] == p.seg_gen) continue;
        const long gsrc = p.cross ? idx : (long)f * p.num_tiles + idx;
        const long row0 = (gsrc / p.num_tiles) * T + (gsrc % p.num_tiles) * p.tile_tokens;
        layer_add_update(p, base + row0 - rel, -1, sn[(size_t)idx]);
        sn[(size_t)idx] = 0;
        sp[(size_t)idx] = -1;
    }
    list.clear();
    for (const Pipeline::Seg& s : segs) {
        sn[(size_t)s.idx] = s.n;
        sp[(size_t)s.idx] = p.tile_phys[(size_t)s.gsrc];
        list.push_back(s.idx);
    }
}

// Frame f's descriptor writes (bf16): the frame's segments encoded per
// 16-row group of its key range, against the entries the device holds.
void layer_gd_collect(Pipeline& p, int f) {
    if (p.gd_stride == 0) return;
    const long T = p.T;
    const long rel = p.cross ? 0 : (long)f * T;
    long b, e;
    frame_range(p, f, b, e);
    p.gd_subs.clear();
    for (const Pipeline::Seg& s : p.frame_segs[(size_t)f]) {
        const long row0 = (s.gsrc / p.num_tiles) * T + (s.gsrc % p.num_tiles) * p.tile_tokens;
        kvp::gd::add_rows(p.gd_subs, row0 - rel, s.n, p.tile_phys[(size_t)s.gsrc], b, e);
    }
    kvp::gd::encode(p.gd_subs, p.gd_new);
    // both lists are in group order: write what changed, clear what is gone
    std::vector<kvp::gd::Ent>& old = p.gd_dev[(size_t)f];
    const long base = (long)f * p.gd_stride;
    size_t i = 0, j = 0;
    while (i < old.size() || j < p.gd_new.size()) {
        if (j == p.gd_new.size() || (i < old.size() && old[i].g < p.gd_new[j].g)) {
            p.gd_writes.push_back(kvp::LayerGdWrite{base + old[i].g, 0u, 0u});
            ++i;
        } else if (i == old.size() || p.gd_new[j].g < old[i].g) {
            p.gd_writes.push_back(kvp::LayerGdWrite{base + p.gd_new[j].g, p.gd_new[j].w0, p.gd_new[j].w1});
            ++j;
        } else {
            if (old[i].w0 != p.gd_new[j].w0 || old[i].w1 != p.gd_new[j].w1)
                p.gd_writes.push_back(
                    kvp::LayerGdWrite{base + p.gd_new[j].g, p.gd_new[j].w0, p.gd_new[j].w1});
            ++i;
            ++j;
        }
    }
    old.swap(p.gd_new);
}

// One attention launch over all frames of the layer (the layer's arena,
// map slices and, in bf16, descriptor tables).
int layer_attention(Pipeline& p, const char* q, const char* k, const char* v, char* out) {
    kvp::AttnLaunch L;
    L.dtype = p.dtype;
    L.q = q;
    L.k = k;
    L.v = v;
    L.out = out;
    if (p.persist) {
        L.arena = p.layer_arena;  // one arena for every frame
        L.kvmap = p.layer_map;
        L.map_fstride = p.map_stride;
        if (!p.cold_rows_nt) {
            L.gdesc = p.layer_gd;
            L.gd_fstride = p.gd_stride;
        }
    }
    L.nq = p.T;
    L.D = p.D;
    L.heads = p.heads;
    L.frames = p.frames;
    L.q_fstride = (long)p.T * p.D;
    L.layer = true;
    L.cold_rows_nt = p.cold_rows_nt;
    L.stream = p.stream;
    if (p.cross) {
        L.key_begin = 0;
        L.key_end = p.T;      // frame 0: [0, T)
        L.kend_step = p.T;    // frame f: ends at (f + 1) * T
        L.max_span = p.window > 0 ? (long)p.window * p.T : 0;
    } else {
        L.kv_fstride = (long)p.T * p.D;
        L.key_begin = 0;
        L.key_end = p.T;
    }
    return kvp::launch_attention(L);
}

// The staging launch of a plan-only layer run, applied on the host: the
// layer map, the descriptor tables and the physical rows' sources. Fails
// when two runs of the launch would write one physical row, one map entry
// or one descriptor entry (the workgroups of one launch run in no fixed
// order).
int layer_apply_host(Pipeline& p) {
    p.plan_src.assign((size_t)p.layer_nphys, -1L);
    for (const kvp::LayerCopyRun& r : p.layer_copies) {
        for (int j = 0; j < r.n; ++j) {
            const long d = (long)r.dst_row + j;
            if (d < 0 || d >= p.layer_nphys || p.plan_src[(size_t)d] >= 0) {
                kvp::set_error("pipeline: copy runs overlap or leave the arena at row %ld", d);
                return 1;
            }
            p.plan_src[(size_t)d] = (long)r.src_row + j;
        }
    }
    const int gen = p.layer_gen;
    for (const kvp::LayerMapRun& m : p.layer_updates) {
        for (int j = 0; j < m.n; ++j) {
            const long e = m.index + j;
            if (e < 0 || e >= (long)p.plan_map.size() || p.plan_stamp[(size_t)e] == gen) {
                kvp::set_error("pipeline: map runs overlap or leave the map at entry %ld", e);
                return 1;
            }
            p.plan_stamp[(size_t)e] = gen;
            p.plan_map[(size_t)e] = m.value < 0 ? -1L : (long)m.value + j;
        }
    }
    std::vector<char> hit(p.plan_gd.size() / 2, 0);
    for (const kvp::LayerGdWrite& w : p.gd_writes) {
        if (w.index < 0 || 2 * w.index >= (long)p.plan_gd.size() || hit[(size_t)w.index]) {
            kvp::set_error("pipeline: descriptor writes overlap or leave the table at %ld", w.index);
            return 1;
        }
        hit[(size_t)w.index] = 1;
        p.plan_gd[(size_t)(2 * w.index)] = w.w0;
        p.plan_gd[(size_t)(2 * w.index + 1)] = w.w1;
    }
    return 0;
}

// A whole layer: host plans of every frame, one staging launch (the copies,
// map runs and descriptor writes), one attention launch. Plan-only
// pipelines apply the staging on the host instead and launch nothing. A
// failure once the host mirrors of the device map and descriptor tables
// have moved on tears the layer state down, so that the next run starts
// from a fresh device map instead of one the mirrors no longer describe.
int run_layer(Pipeline& p, const char* q, const char* k, const char* v, char* out,
              const float* scores_flat) {
    p.next_frame = 0;
    if (!check_data(p, q, k, v, out)) return 1;
    if (!p.persist) {
        p.count = 0;
        p.staged_tiles = 0;
        p.copy_rows = 0;
        return p.plan_only ? 0 : layer_attention(p, q, k, v, out);
    }
    if (layer_setup(p)) return 1;
    p.last_mgr = p.layer_mgr.get();
    ++p.layer_gen;
    p.layer_nphys = 0;
    p.layer_copies.clear();
    p.layer_updates.clear();
    p.gd_writes.clear();
    for (int f = 0; f < p.frames; ++f) {
        if (select_and_release(p, *p.layer_mgr, f, scores_flat)) return 1;
        plan_frame_layer(p, *p.layer_mgr, f, k, v);
        finish_frame(p, *p.layer_mgr, f);
    }
    if (layer_assign(p)) return 1;
    for (int f = 0; f < p.frames; ++f) {
        layer_collect(p, f);
        layer_gd_collect(p, f);
    }
    int rc = p.plan_only
                 ? layer_apply_host(p)
                 : kvp::layer_stage_launch(p.layer_stager, p.layer_arena, k, v,
                                           (long)p.D * p.elem, p.layer_copies.data(),
                                           (long)p.layer_copies.size(), p.layer_map,
                                           p.layer_updates.data(), (long)p.layer_updates.size(),
                                           p.layer_gd, p.gd_writes.data(),
                                           (long)p.gd_writes.size(), p.stream);
    if (rc == 0 && !p.plan_only) rc = layer_attention(p, q, k, v, out);
    if (rc) {
        const std::string err = kvp_last_error();
        layer_teardown(p);
        kvp::set_error("%s", err.c_str());
    }
    return rc;
}

}  // namespace

extern "C" {

void* kvp_pipeline_create(const char* policy, int cross, int streaming, int frames, int T,
                          int D, int heads, int tile_tokens, long set_aside_bytes, int dtype,
                          int window_frames, int plan_only) {
    if (!policy || frames <= 0 || T <= 0 || heads <= 0 || D != heads * 128 ||
        tile_tokens <= 0 || (dtype != 0 && dtype != 1) || window_frames < 0) {
        kvp::set_error("pipeline: bad arguments");
        return nullptr;
    }
    std::unique_ptr<Pipeline> p(new (std::nothrow) Pipeline());
    if (!p) return nullptr;
    p->num_tiles = (T + tile_tokens - 1) / tile_tokens;
    p->policy.reset(make_tile_gating_policy(policy, (int)p->num_tiles, frames));
    if (!p->policy) {
        kvp::set_error("pipeline: unknown policy %s", policy);
        return nullptr;
    }
    p->persist = strcmp(policy, "none") != 0;
    p->cross = cross != 0;
    p->streaming = streaming != 0 && p->persist;
    p->plan_only = plan_only != 0;
    p->frames = frames;
    p->T = T;
    p->D = D;
    p->heads = heads;
    p->tile_tokens = tile_tokens;
    p->window = window_frames;
    p->dtype = dtype;
    p->elem = dtype == 1 ? 2 : 4;
    p->set_aside = set_aside_bytes;
    // slots = set_aside / (tile_tokens * hidden * elem * 2)
    // (reference: src/run_policy_experiment.cu:143-144, fp32 there).
    const long tile_bytes = (long)tile_tokens * D * p->elem * 2;
    p->slots = set_aside_bytes > 0 ? set_aside_bytes / tile_bytes : 0;
    p->ids.assign((size_t)std::max<long>((long)frames * p->num_tiles, p->slots) + 1, 0);
    if (p->persist) {
        if (set_aside_bytes <= 0) {
            kvp::set_error("pipeline: policy %s needs a positive set-aside", policy);
            return nullptr;
        }
        p->mgr.reset(new KVTileManager((size_t)set_aside_bytes, (size_t)set_aside_bytes));
        const size_t stride_floats = (size_t)D * 2 * p->elem / sizeof(float);
        const bool ok = p->mgr->init() &&
                        (p->plan_only
                             ? p->mgr->arena_attach(nullptr, (size_t)set_aside_bytes, stride_floats)
                             : p->mgr->arena_init((size_t)set_aside_bytes, stride_floats));
        if (!ok) {
            kvp::set_error("pipeline: manager init failed");
            return nullptr;
        }
        p->h_map.assign((size_t)frames * T, -1L);
        if (!p->plan_only) {
            const size_t n = (size_t)frames * T;
            p->d_map = static_cast<long*>(kvp_dev_alloc(n * sizeof(long)));
            if (!p->d_map) return nullptr;
            p->dev_mirror.assign(n, -1L);
            p->stamp.assign(n, 0);
            // the device map starts as all -1, matching the mirror
            if (!p->mgr->flush_with_map(p->d_map, (long)n, nullptr, nullptr, 0)) return nullptr;
        }
    }
    return p.release();
}

void kvp_pipeline_destroy(void* p) { delete PL(p); }

int kvp_pipeline_set_stream(void* p, void* stream) {
    PL(p)->stream = stream;
    if (PL(p)->mgr) PL(p)->mgr->set_stream(stream);
    return 0;
}

int kvp_pipeline_set_cold_rows_nt(void* p, int on) {
    PL(p)->cold_rows_nt = on != 0;
    return 0;
}

int kvp_pipeline_step(void* p, int f, const void* q, const void* k, const void* v, void* out,
                      const float* scores_flat) {
    Pipeline& pl = *PL(p);
    if (f < 0 || f >= pl.frames) {
        kvp::set_error("pipeline: frame %d out of range", f);
        return 1;
    }
    return step_frame(pl, f, static_cast<const char*>(q), static_cast<const char*>(k),
                      static_cast<const char*>(v), static_cast<char*>(out), scores_flat);
}

int kvp_pipeline_run(void* p, const void* q, const void* k, const void* v, void* out,
                     const float* scores_flat) {
    return run_layer(*PL(p), static_cast<const char*>(q), static_cast<const char*>(k),
                     static_cast<const char*>(v), static_cast<char*>(out), scores_flat);
}

int kvp_pipeline_selected(void* p, long* ids, int cap) {
    Pipeline& pl = *PL(p);
    const int n = std::min(pl.count, cap);
    for (int i = 0; i < n; ++i) ids[i] = pl.ids[i];
    return pl.count;
}

long kvp_pipeline_map(void* p, long* out, long cap) {
    Pipeline& pl = *PL(p);
    const long n = std::min((long)pl.h_map.size(), cap);
    if (n > 0) memcpy(out, pl.h_map.data(), (size_t)n * sizeof(long));
    return (long)pl.h_map.size();
}

long kvp_pipeline_slots(void* p) { return PL(p)->slots; }
long kvp_pipeline_staged_tiles(void* p) { return PL(p)->staged_tiles; }
long kvp_pipeline_staged_bytes(void* p) {
    return PL(p)->last_mgr ? (long)PL(p)->last_mgr->streaming_staged_bytes() : 0;
}
long kvp_pipeline_copy_rows(void* p) { return PL(p)->copy_rows; }
void* kvp_pipeline_arena(void* p) {
    return PL(p)->mgr ? PL(p)->mgr->arena_device_ptr() : nullptr;
}
const long* kvp_pipeline_device_map(void* p) { return PL(p)->d_map; }
void* kvp_pipeline_layer_arena(void* p) { return PL(p)->layer_arena; }
const long* kvp_pipeline_layer_map(void* p) { return PL(p)->layer_map; }
long kvp_pipeline_layer_map_stride(void* p) { return PL(p)->map_stride; }
long kvp_pipeline_layer_copied_rows(void* p) { return PL(p)->layer_nphys; }
long kvp_pipeline_layer_arena_bytes(void* p) {
    const Pipeline& pl = *PL(p);
    return pl.layer_arena ? pl.layer_cap * 2L * pl.D * pl.elem : 0;
}
const unsigned* kvp_pipeline_layer_gd(void* p) { return PL(p)->layer_gd; }
long kvp_pipeline_layer_gd_stride(void* p) { return PL(p)->gd_stride; }

int kvp_pipeline_layer_attention(void* p, const void* q, const void* k, const void* v,
                                 void* out) {
    Pipeline& pl = *PL(p);
    if (pl.plan_only || (pl.persist && !pl.layer_arena)) {
        kvp::set_error("pipeline: no layer run to repeat");
        return 1;
    }
    if (!check_data(pl, static_cast<const char*>(q), static_cast<const char*>(k),
                    static_cast<const char*>(v), static_cast<const char*>(out)))
        return 1;
    return layer_attention(pl, static_cast<const char*>(q), static_cast<const char*>(k),
                           static_cast<const char*>(v), static_cast<char*>(out));
}

long kvp_pipeline_layer_plan_gd(void* p, int f, unsigned* out, long cap) {
    const Pipeline& pl = *PL(p);
    if (!pl.plan_only || f < 0 || f >= pl.frames || pl.plan_gd.empty()) return -1;
    const long n = std::min(pl.gd_stride, cap);
    if (n > 0)
        memcpy(out, pl.plan_gd.data() + (size_t)f * 2 * pl.gd_stride, (size_t)n * 2 * sizeof(unsigned));
    return pl.gd_stride;
}

long kvp_pipeline_layer_plan_map(void* p, int f, long* out, long cap) {
    const Pipeline& pl = *PL(p);
    if (!pl.plan_only || f < 0 || f >= pl.frames || pl.plan_map.empty()) return -1;
    const long n = std::min(pl.map_stride, cap);
    if (n > 0) memcpy(out, pl.plan_map.data() + (size_t)f * pl.map_stride, (size_t)n * sizeof(long));
    return pl.map_stride;
}

long kvp_pipeline_layer_plan_sources(void* p, long* out, long cap) {
    const Pipeline& pl = *PL(p);
    if (!pl.plan_only) return -1;
    const long n = std::min((long)pl.plan_src.size(), cap);
    if (n > 0) memcpy(out, pl.plan_src.data(), (size_t)n * sizeof(long));
    return (long)pl.plan_src.size();
}
void* kvp_pipeline_manager(void* p) { return PL(p)->mgr.get(); }

}  // extern "C"
