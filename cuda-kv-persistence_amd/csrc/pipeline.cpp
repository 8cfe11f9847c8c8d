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
//   4. one flush = one launch: every row copy plus the KVMap entries that
//      change (rows leaving the pinned set -> -1, new or moved rows -> slot);
//   5. one attention launch for the frame.
// The device KVMap is never rebuilt from scratch: a host mirror of it gives
// the exact difference to the map the reference driver would upload for this
// frame (prefix reset to -1, then the staged rows), so after step 4 the
// device map holds that map on the whole prefix (and -1 beyond it).
// Nothing synchronises the host per frame: staging, map updates and
// attention are ordered on the pipeline's stream. kvp_pipeline_step runs
// steps 1-5 for one frame in that order; kvp_pipeline_run plans frame f+1
// before launching frame f and has frame f's attention launch carry frame
// f+1's staging (as trailing workgroups of its split-combine launch, or as
// the launch right after it), which saves one launch per frame. The staging
// of frame f+1 still runs after frame f's attention has read the arena and
// the map, so device results are those of frame-by-frame stepping.

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

    ~Pipeline() {
        mgr.reset();
        if (d_map) {
            kvp_stream_sync(stream);
            kvp_dev_free(d_map);
        }
    }
};

Pipeline* PL(void* p) { return static_cast<Pipeline*>(p); }

long window_first_frame(const Pipeline& p, int f) {
    return (p.cross && p.window > 0 && f + 1 > p.window) ? f + 1 - p.window : 0;
}

// Steps 1-4 of a gated frame: selection, streaming release, staging and the
// KVMap difference, prepared as one staging plan (*plan; launched by the
// caller, not here). Host bookkeeping only.
int plan_frame(Pipeline& p, int f, const char* k, const char* v, const float* scores_flat, void** plan) {
    *plan = nullptr;
    const long T = p.T;
    const long row_bytes = (long)p.D * p.elem;
    if (!scores_flat) {
        kvp::set_error("pipeline: policy %s needs motion scores", p.policy->name());
        return 1;
    }
    const long kb_frame = window_first_frame(p, f);

    KVTileManager& mgr = *p.mgr;
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

// Step 5: the frame's attention launch, followed on the stream by the
// staging plan `follow` (may be null).
int launch_frame(Pipeline& p, int f, const char* q, const char* k, const char* v, char* out,
                 const void* follow) {
    const long T = p.T;
    const long frame_bytes = T * (long)p.D * p.elem;
    const long kb_frame = window_first_frame(p, f);
    const void* arena = p.persist ? p.mgr->arena_device_ptr() : nullptr;
    const long* map = p.persist ? p.d_map : nullptr;
    if (p.cross)
        return kvp::launch_attention(p.dtype, q + f * frame_bytes, k, v, arena, map,
                                     out + f * frame_bytes, p.T, p.D, p.heads, 1, 0, 0, 0,
                                     kb_frame * T, (long)(f + 1) * T, p.stream, follow);
    return kvp::launch_attention(p.dtype, q + f * frame_bytes, k + f * frame_bytes,
                                 v + f * frame_bytes, arena, map ? map + (long)f * T : nullptr,
                                 out + f * frame_bytes, p.T, p.D, p.heads, 1, 0, 0, 0, 0, T, p.stream,
                                 follow);
}

// Step 6: end of the frame's step in the manager.
void finish_frame(Pipeline& p, int f) {
    if (p.streaming)
        p.prev_selected = p.selected;
    else
        p.mgr->arena_end_step();
    if (p.streaming && f + 1 == p.frames) p.mgr->streaming_end();
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
        return launch_frame(p, f, q, k, v, out, nullptr);
    }
    void* plan = nullptr;
    int rc = plan_frame(p, f, k, v, scores_flat, &plan);
    if (rc == 0 && plan) rc = kvp::stage_plan_launch(plan, p.stream);
    kvp::stage_plan_free(plan);
    if (rc == 0 && !p.plan_only) rc = launch_frame(p, f, q, k, v, out, nullptr);
    if (rc) return rc;
    finish_frame(p, f);
    p.next_frame = (f + 1 == p.frames) ? 0 : f + 1;
    return 0;
}

// All frames, the staging of frame f+1 carried by frame f's attention
// launch: frame f+1 is planned (host bookkeeping) before frame f's launch,
// and its copies and map updates run right after frame f's attention on the
// stream, as trailing workgroups of its split-combine launch when there is
// one. Device results equal frame-by-frame stepping.
int run_frames(Pipeline& p, const char* q, const char* k, const char* v, char* out,
               const float* scores_flat) {
    p.next_frame = 0;
    if (!p.persist || p.plan_only) {
        for (int f = 0; f < p.frames; ++f) {
            const int rc = step_frame(p, f, q, k, v, out, scores_flat);
            if (rc) return rc;
        }
        return 0;
    }
    if (!check_data(p, q, k, v, out)) return 1;
    void* plan = nullptr;
    int rc = plan_frame(p, 0, k, v, scores_flat, &plan);
    if (rc == 0 && plan) rc = kvp::stage_plan_launch(plan, p.stream);
    kvp::stage_plan_free(plan);
    for (int f = 0; rc == 0 && f < p.frames; ++f) {
        finish_frame(p, f);
        void* next = nullptr;
        if (f + 1 < p.frames) rc = plan_frame(p, f + 1, k, v, scores_flat, &next);
        if (rc == 0) rc = launch_frame(p, f, q, k, v, out, next);
        kvp::stage_plan_free(next);
    }
    p.next_frame = 0;
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
    return run_frames(*PL(p), static_cast<const char*>(q), static_cast<const char*>(k),
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
void* kvp_pipeline_manager(void* p) { return PL(p)->mgr.get(); }

}  // extern "C"
