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
//     decisions); frame f's arena state goes to its own region of a layer
//     arena (every mapped row copied to region f at its slot) and frame f's
//     KVMap to its own slice of a layer map, all in one staging launch; then
//     one attention launch covers every frame, each reading its own region
//     and slice. Region f holds, at every slot frame f's map points to, what
//     the single arena holds at frame f, so the outputs are those of
//     frame-by-frame stepping, bit for bit.
// Nothing synchronises the host per frame; all device work is ordered on the
// pipeline's stream.

#include <algorithm>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

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
    char* layer_arena = nullptr;               // frames regions of region_bytes
    long region_rows = 0, region_bytes = 0;
    long* layer_map = nullptr;                 // frames slices of map_stride entries
    long map_stride = 0;
    std::vector<long> layer_mirror;            // device content of layer_map
    std::vector<std::vector<long>> layer_rows; // per frame: rows mapped on the device
    std::vector<int> layer_stamp;
    int layer_step = 0;
    std::vector<KvpRowCopy> layer_copies;
    void* layer_stager = nullptr;

    ~Pipeline() {
        mgr.reset();
        layer_mgr.reset();
        if (d_map || layer_arena || layer_map || layer_stager) kvp_stream_sync(stream);
        if (layer_stager) kvp_stager_destroy(layer_stager);
        if (d_map) kvp_dev_free(d_map);
        if (layer_arena) kvp_dev_free(layer_arena);
        if (layer_map) kvp_dev_free(layer_map);
    }
};

Pipeline* PL(void* p) { return static_cast<Pipeline*>(p); }

long window_first_frame(const Pipeline& p, int f) {
    return (p.cross && p.window > 0 && f + 1 > p.window) ? f + 1 - p.window : 0;
}

// Steps 1-3 of a gated frame on manager `mgr`: selection, streaming release
// and staging, leaving the frame's mapped rows in p.map_rows / p.map_slots
// and its host map in p.h_map. Host bookkeeping only (a manager with a device
// arena records its copies for the next flush).
int plan_frame_host(Pipeline& p, KVTileManager& mgr, int f, const char* k, const char* v,
                    const float* scores_flat) {
    const long T = p.T;
    const long row_bytes = (long)p.D * p.elem;
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

// Layer-mode device state, created at the first kvp_pipeline_run.
int layer_setup(Pipeline& p) {
    if (p.layer_mgr) return 0;
    const long row_bytes = (long)p.D * p.elem;
    const size_t stride_floats = (size_t)2 * row_bytes / sizeof(float);
    p.layer_mgr.reset(new (std::nothrow) KVTileManager((size_t)p.set_aside, (size_t)p.set_aside));
    if (!p.layer_mgr || !p.layer_mgr->init() ||
        !p.layer_mgr->arena_attach(nullptr, (size_t)p.set_aside, stride_floats)) {
        p.layer_mgr.reset();
        kvp::set_error("pipeline: layer manager init failed");
        return 1;
    }
    p.region_rows = p.set_aside / (2 * row_bytes);
    p.region_bytes = p.region_rows * 2 * row_bytes;
    p.map_stride = p.cross ? (long)p.frames * p.T : (long)p.T;
    const long map_entries = (long)p.frames * p.map_stride;
    p.layer_arena = static_cast<char*>(
        kvp_dev_alloc((size_t)std::max<long>(1, p.frames * p.region_bytes)));
    p.layer_map = static_cast<long*>(kvp_dev_alloc((size_t)map_entries * sizeof(long)));
    p.layer_stager = kvp_stager_create();
    if (!p.layer_arena || !p.layer_map || !p.layer_stager) {
        kvp::set_error("pipeline: layer arena / map allocation failed");
        return 1;
    }
    p.layer_mirror.assign((size_t)map_entries, -1L);
    p.layer_rows.assign((size_t)p.frames, {});
    p.layer_stamp.assign((size_t)p.map_stride, 0);
    // the device map starts as all -1, matching the mirror
    if (kvp_stage_run(p.layer_stager, nullptr, 0, nullptr, 0, p.layer_map, map_entries, nullptr,
                      nullptr, 0, p.stream))
        return 1;
    return 0;
}

// Frame f's share of the layer staging launch: every mapped row copied into
// region f at its slot, and the entries of map slice f that change.
void layer_collect(Pipeline& p, int f, const char* k, const char* v) {
    const long row_bytes = (long)p.D * p.elem;
    const long base = (long)f * p.map_stride;
    const long rel = p.cross ? 0 : (long)f * p.T;  // intra slices are frame-relative
    ++p.layer_step;
    for (size_t i = 0; i < p.map_rows.size(); ++i) {
        const long r = p.map_rows[i];
        const long slot = p.map_slots[i];
        KvpRowCopy c;
        c.k_src = k + r * row_bytes;
        c.v_src = v + r * row_bytes;
        c.dst_row = (long)f * p.region_rows + slot;
        c.k_bytes = (unsigned)row_bytes;
        c.v_bytes = (unsigned)row_bytes;
        p.layer_copies.push_back(c);
        const long e = r - rel;
        p.layer_stamp[(size_t)e] = p.layer_step;
        if (p.layer_mirror[(size_t)(base + e)] != slot) {
            p.upd_rows.push_back(base + e);
            p.upd_vals.push_back(slot);
            p.layer_mirror[(size_t)(base + e)] = slot;
        }
    }
    std::vector<long>& prev = p.layer_rows[(size_t)f];
    for (long e : prev) {
        if (p.layer_stamp[(size_t)e] != p.layer_step && p.layer_mirror[(size_t)(base + e)] != -1) {
            p.upd_rows.push_back(base + e);
            p.upd_vals.push_back(-1);
            p.layer_mirror[(size_t)(base + e)] = -1;
        }
    }
    prev.clear();
    for (long r : p.map_rows) prev.push_back(r - rel);
}

// One attention launch over all frames of the layer.
int layer_attention(Pipeline& p, const char* q, const char* k, const char* v, char* out) {
    kvp::AttnLaunch L;
    L.dtype = p.dtype;
    L.q = q;
    L.k = k;
    L.v = v;
    L.out = out;
    if (p.persist) {
        L.arena = p.layer_arena;
        L.kvmap = p.layer_map;
        L.map_fstride = p.map_stride;
        L.arena_fstride = p.region_bytes;
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

// A whole layer: host plans of every frame, one staging launch for all
// frames' arena regions and map slices, one attention launch.
int run_layer(Pipeline& p, const char* q, const char* k, const char* v, char* out,
              const float* scores_flat) {
    p.next_frame = 0;
    if (p.plan_only) {
        for (int f = 0; f < p.frames; ++f) {
            const int rc = step_frame(p, f, q, k, v, out, scores_flat);
            if (rc) return rc;
        }
        return 0;
    }
    if (!check_data(p, q, k, v, out)) return 1;
    if (!p.persist) {
        p.count = 0;
        p.staged_tiles = 0;
        p.copy_rows = 0;
        return layer_attention(p, q, k, v, out);
    }
    if (layer_setup(p)) return 1;
    p.layer_copies.clear();
    p.upd_rows.clear();
    p.upd_vals.clear();
    for (int f = 0; f < p.frames; ++f) {
        if (plan_frame_host(p, *p.layer_mgr, f, k, v, scores_flat)) return 1;
        layer_collect(p, f, k, v);
        finish_frame(p, *p.layer_mgr, f);
    }
    if (!p.layer_copies.empty() || !p.upd_rows.empty()) {
        if (kvp_stage_run(p.layer_stager, p.layer_arena, 2L * p.D * p.elem, p.layer_copies.data(),
                          (long)p.layer_copies.size(), p.layer_map, 0, p.upd_rows.data(),
                          p.upd_vals.data(), (long)p.upd_rows.size(), p.stream))
            return 1;
    }
    return layer_attention(p, q, k, v, out);
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
    return PL(p)->mgr ? (long)PL(p)->mgr->streaming_staged_bytes() : 0;
}
long kvp_pipeline_copy_rows(void* p) { return PL(p)->copy_rows; }
void* kvp_pipeline_arena(void* p) {
    return PL(p)->mgr ? PL(p)->mgr->arena_device_ptr() : nullptr;
}
const long* kvp_pipeline_device_map(void* p) { return PL(p)->d_map; }
void* kvp_pipeline_layer_arena(void* p) { return PL(p)->layer_arena; }
long kvp_pipeline_layer_region_bytes(void* p) { return PL(p)->region_bytes; }
const long* kvp_pipeline_layer_map(void* p) { return PL(p)->layer_map; }
long kvp_pipeline_layer_map_stride(void* p) { return PL(p)->map_stride; }
void* kvp_pipeline_manager(void* p) { return PL(p)->mgr.get(); }

}  // extern "C"
