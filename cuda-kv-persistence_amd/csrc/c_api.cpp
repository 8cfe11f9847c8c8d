// extern "C" facade of libkvpersist.so (host C++, g++).
//   kvtm_*          : KVTileManager facade, same symbols and return values as
//                     the reference ctypes contract
//                     (reference: src/kv_tile_manager.cu:223-341)
//   kvp_policy_*    : TileGatingPolicy objects
//   kvp_attn_*      : attention entry points (reference signatures of
//                     src/attn_kernel.h:15-29 plus bf16 / window forms)
// plus the C++-linkage attn_forward_launcher / attn_forward_single_frame.

#include <new>

#include "attn_kernel.h"
#include "kv_tile_manager.h"
#include "kvp_c_api.h"
#include "group_desc.h"
#include "kvp_internal.h"
#include "tile_gating_policy.h"
#include "tile_layout.h"

namespace {
KVTileManager* M(void* m) { return static_cast<KVTileManager*>(m); }
TileGatingPolicy* P(void* p) { return static_cast<TileGatingPolicy*>(p); }

constexpr int kHeadDim = 128;
}  // namespace

extern "C" {

// ---- KVTileManager facade ----

void* kvtm_create(long budget_bytes, long max_window_bytes) {
    try {
        return new KVTileManager((size_t)budget_bytes, (size_t)max_window_bytes);
    } catch (...) {
        return nullptr;
    }
}

void kvtm_destroy(void* m) { delete M(m); }
int kvtm_init(void* m) { return M(m)->init() ? 1 : 0; }
long kvtm_query_limit(void* m) { return (long)M(m)->query_device_limit(); }
int kvtm_admit(void* m, long tile_id, void* ptr, long bytes) {
    if (bytes < 0) return (int)KVTM_INVALID;
    return (int)M(m)->admit(tile_id, ptr, (size_t)bytes);
}
int kvtm_release(void* m, long tile_id) { return M(m)->release(tile_id) ? 1 : 0; }
void kvtm_clear(void* m) { M(m)->clear(); }
long kvtm_persisted_bytes(void* m) { return (long)M(m)->persisted_bytes(); }
int kvtm_persisted_tiles(void* m) { return M(m)->persisted_tiles(); }

void* kvtm_dev_alloc(long bytes) {
    if (bytes <= 0) return nullptr;
    return kvp_dev_alloc((size_t)bytes);
}
void kvtm_dev_free(void* p) { kvp_dev_free(p); }

int kvtm_arena_init(void* m, long cap_bytes, long row_stride_floats) {
    if (cap_bytes <= 0 || row_stride_floats <= 0) return 0;
    return M(m)->arena_init((size_t)cap_bytes, (size_t)row_stride_floats) ? 1 : 0;
}
void kvtm_arena_begin(void* m) { M(m)->arena_begin_step(); }
int kvtm_arena_stage(void* m, const void* k_dev, long k_bytes, const void* v_dev,
                     long v_bytes, long* out_row) {
    if (k_bytes < 0 || v_bytes < 0 || !out_row) return 0;
    return M(m)->arena_stage(k_dev, (size_t)k_bytes, v_dev, (size_t)v_bytes, out_row) ? 1 : 0;
}
int kvtm_arena_window(void* m) { return M(m)->arena_apply_window() ? 1 : 0; }
void kvtm_arena_end(void* m) { M(m)->arena_end_step(); }
long kvtm_arena_used(void* m) { return (long)M(m)->arena_used_bytes(); }
void* kvtm_arena_ptr(void* m) { return M(m)->arena_device_ptr(); }

int kvtm_streaming_begin(void* m) { return M(m)->streaming_begin() ? 1 : 0; }
int kvtm_streaming_stage(void* m, long row_id, const void* k_dev, long k_bytes,
                         const void* v_dev, long v_bytes, int changed,
                         long* out_slot, int* restaged) {
    bool r = false;
    long slot = -1;
    int ok = 0;
    if (k_bytes >= 0 && v_bytes >= 0)
        ok = M(m)->streaming_stage(row_id, k_dev, (size_t)k_bytes, v_dev,
                                   (size_t)v_bytes, changed != 0, &slot, &r) ? 1 : 0;
    if (out_slot) *out_slot = slot;
    if (restaged) *restaged = r ? 1 : 0;
    return ok;
}
int kvtm_streaming_release(void* m, long row_id) {
    return M(m)->streaming_release(row_id) ? 1 : 0;
}
int kvtm_streaming_window(void* m) { return M(m)->streaming_apply_window() ? 1 : 0; }
void kvtm_streaming_end(void* m) { M(m)->streaming_end(); }
long kvtm_streaming_staged_bytes(void* m) { return (long)M(m)->streaming_staged_bytes(); }

long kvtm_layout_tiles_per_frame(int tokens_per_frame, int tile_tokens) {
    return TileLayout(tokens_per_frame, tile_tokens).tiles_per_frame;
}
long kvtm_layout_tile_start(int tpf, int tt, long id) {
    return TileLayout(tpf, tt).tile_start(id);
}
int kvtm_layout_tile_count(int tpf, int tt, long id) {
    return TileLayout(tpf, tt).tile_count(id);
}

int kvtm_arena_attach(void* m, void* dev_ptr, long cap_bytes, long row_stride_floats) {
    if (cap_bytes <= 0 || row_stride_floats <= 0) return 0;
    return M(m)->arena_attach(dev_ptr, (size_t)cap_bytes, (size_t)row_stride_floats) ? 1 : 0;
}
int kvtm_flush(void* m) { return M(m)->flush() ? 1 : 0; }
void kvtm_set_stream(void* m, void* stream) { M(m)->set_stream(stream); }
int kvtm_is_persisted(void* m, long tile_id) { return M(m)->is_persisted(tile_id) ? 1 : 0; }
long kvtm_streaming_high_water(void* m) { return M(m)->streaming_high_water(); }
long kvtm_streaming_capacity(void* m) { return M(m)->streaming_capacity_rows(); }
long kvtm_pending_copies(void* m) { return (long)M(m)->pending_copies(); }

// ---- policies ----

void* kvp_policy_create(const char* name, int tiles_per_frame, int total_frames) {
    try {
        return make_tile_gating_policy(name, tiles_per_frame, total_frames);
    } catch (...) {
        return nullptr;
    }
}
void kvp_policy_destroy(void* p) { delete P(p); }
const char* kvp_policy_name(void* p) { return P(p)->name(); }
int kvp_policy_select(void* p, const float* scores, int num_candidates, int max_tiles,
                      long* out_ids) {
    int count = 0;
    P(p)->select(scores, num_candidates, max_tiles, out_ids, &count);
    return count;
}
int kvp_policy_select_range(void* p, const float* scores_flat, long first_id,
                            int num_candidates, int max_tiles, long* out_ids) {
    int count = 0;
    P(p)->select_range(scores_flat, first_id, num_candidates, max_tiles, out_ids, &count);
    return count;
}

// ---- attention ----

// reference: src/gated_attention_kernel.cu:141-168. remap=true runs the
// per-frame intra launches with the map sliced per frame; remap=false runs
// identity addressing. Both are one launch here with frames in the grid.
int kvp_attn_forward_launcher(const float* d_q, const float* d_k, const float* d_v,
                              const float* d_arena, const long* d_kvmap, float* d_out,
                              int frames, int T, int D, int heads, int remap) {
    const long TD = (long)T * D;
    return kvp::launch_attention(0, d_q, d_k, d_v, remap ? d_arena : nullptr,
                                 remap ? d_kvmap : nullptr, d_out, T, D, heads, frames,
                                 TD, TD, T, 0, T, kvp::library_stream());
}

int kvp_attn_forward_launcher_bf16(const void* d_q, const void* d_k, const void* d_v,
                                   const void* d_arena, const long* d_kvmap, void* d_out,
                                   int frames, int T, int D, int heads, int remap) {
    const long TD = (long)T * D;
    return kvp::launch_attention(1, d_q, d_k, d_v, remap ? d_arena : nullptr,
                                 remap ? d_kvmap : nullptr, d_out, T, D, heads, frames,
                                 TD, TD, T, 0, T, kvp::library_stream());
}

static int single_frame(int dtype, const void* q_f, const void* k, const void* v,
                        const void* arena, const long* kvmap_f, void* out_f, int T, int D,
                        int heads, int cross, int frame_idx, int window_frames) {
    if (T <= 0 || frame_idx < 0 || window_frames < 0) {
        kvp::set_error("attention: bad frame arguments (T=%d frame=%d window=%d)", T,
                       frame_idx, window_frames);
        return 1;
    }
    long kb = 0, ke = T;
    if (cross) {
        ke = (long)(frame_idx + 1) * T;
        if (window_frames > 0 && frame_idx + 1 > window_frames)
            kb = (long)(frame_idx + 1 - window_frames) * T;
    }
    return kvp::launch_attention(dtype, q_f, k, v, arena, kvmap_f, out_f, T, D, heads, 1, 0,
                                 0, 0, kb, ke, kvp::library_stream());
}

// reference: src/gated_attention_kernel.cu:170-184
int kvp_attn_forward_single_frame(const float* d_q_f, const float* d_k, const float* d_v,
                                  const float* d_arena, const long* d_kvmap_f,
                                  float* d_out_f, int T, int D, int heads, int cross,
                                  int frame_idx) {
    return single_frame(0, d_q_f, d_k, d_v, d_arena, d_kvmap_f, d_out_f, T, D, heads, cross,
                        frame_idx, 0);
}

int kvp_attn_forward_single_frame_window(const float* d_q_f, const float* d_k,
                                         const float* d_v, const float* d_arena,
                                         const long* d_kvmap_f, float* d_out_f, int T,
                                         int D, int heads, int cross, int frame_idx,
                                         int window_frames) {
    return single_frame(0, d_q_f, d_k, d_v, d_arena, d_kvmap_f, d_out_f, T, D, heads, cross,
                        frame_idx, window_frames);
}

int kvp_attn_forward_single_frame_bf16(const void* d_q_f, const void* d_k, const void* d_v,
                                       const void* d_arena, const long* d_kvmap_f,
                                       void* d_out_f, int T, int D, int heads, int cross,
                                       int frame_idx, int window_frames) {
    return single_frame(1, d_q_f, d_k, d_v, d_arena, d_kvmap_f, d_out_f, T, D, heads, cross,
                        frame_idx, window_frames);
}

int kvp_attn_forward_range(int dtype, const void* q, const void* k, const void* v,
                           const void* arena, const long* kvmap, void* out, int nq, int D,
                           int heads, long key_begin, long key_end, void* stream) {
    return kvp::launch_attention(dtype, q, k, v, arena, kvmap, out, nq, D, heads, 1, 0, 0, 0,
                                 key_begin, key_end, stream);
}

int kvp_attn_forward_range_noalloc(int dtype, const void* q, const void* k, const void* v,
                                   const void* arena, const long* kvmap, void* out, int nq, int D,
                                   int heads, long key_begin, long key_end, void* stream) {
    kvp::AttnLaunch L;
    L.dtype = dtype;
    L.q = q;
    L.k = k;
    L.v = v;
    L.arena = arena;
    L.kvmap = kvmap;
    L.out = out;
    L.nq = nq;
    L.D = D;
    L.heads = heads;
    L.key_begin = key_begin;
    L.key_end = key_end;
    L.stream = stream;
    return kvp::launch_attention_noalloc(L);
}

}  // extern "C"

// A layer launch of kvp_attn_forward_frames(_gd).
static int forward_frames(int dtype, const void* q, const void* k, const void* v,
                          const void* arena, long arena_frame_bytes, const long* kvmap,
                          long map_frame_stride, const unsigned* gdesc, long gd_frame_stride,
                          void* out, int frames, int T, int D, int heads, int cross,
                          int window_frames, int flags, void* stream) {
    if (T <= 0 || frames <= 0 || window_frames < 0 || arena_frame_bytes < 0 ||
        map_frame_stride < 0) {
        kvp::set_error("attention: bad layer arguments (T=%d frames=%d window=%d)", T, frames,
                       window_frames);
        return 1;
    }
    kvp::AttnLaunch L;
    L.gdesc = gdesc;
    L.gd_fstride = gd_frame_stride;
    L.dtype = dtype;
    L.q = q;
    L.k = k;
    L.v = v;
    L.arena = arena;
    L.kvmap = kvmap;
    L.out = out;
    L.nq = T;
    L.D = D;
    L.heads = heads;
    L.frames = frames;
    L.q_fstride = (long)T * D;
    L.map_fstride = map_frame_stride;
    L.arena_fstride = arena_frame_bytes;
    L.key_begin = 0;
    L.key_end = T;
    L.layer = true;
    L.cold_rows_nt = (flags & KVP_ATTN_COLD_ROWS_NT) != 0;
    L.stream = stream;
    if (cross) {
        L.kend_step = T;
        L.max_span = window_frames > 0 ? (long)window_frames * T : 0;
    } else {
        L.kv_fstride = (long)T * D;
    }
    return kvp::launch_attention(L);
}

extern "C" {

int kvp_attn_forward_frames(int dtype, const void* q, const void* k, const void* v,
                            const void* arena, long arena_frame_bytes, const long* kvmap,
                            long map_frame_stride, void* out, int frames, int T, int D,
                            int heads, int cross, int window_frames, int flags, void* stream) {
    return forward_frames(dtype, q, k, v, arena, arena_frame_bytes, kvmap, map_frame_stride,
                          nullptr, 0, out, frames, T, D, heads, cross, window_frames, flags,
                          stream);
}

int kvp_attn_forward_frames_gd(const void* q, const void* k, const void* v, const void* arena,
                               long arena_frame_bytes, const long* kvmap, long map_frame_stride,
                               const unsigned* gdesc, long gd_frame_stride, void* out,
                               int frames, int T, int D, int heads, int cross, int window_frames,
                               void* stream) {
    if (!gdesc) {
        kvp::set_error("attention: null group-descriptor table");
        return 1;
    }
    return forward_frames(1, q, k, v, arena, arena_frame_bytes, kvmap, map_frame_stride, gdesc,
                          gd_frame_stride, out, frames, T, D, heads, cross, window_frames, 0,
                          stream);
}

long kvp_attn_group_desc(const long* map, long key_begin, long key_end, int D, unsigned* out,
                         long cap) {
    if (!map || key_begin < 0 || key_end <= key_begin || D <= 0 || cap < 0 ||
        (cap > 0 && !out)) {
        kvp::set_error("group descriptors: bad arguments");
        return -1;
    }
    const long n = 4 * ((key_end - key_begin + 63) / 64);
    if (cap < n) return n;
    // an entry counts when its arena row lies within the bf16 kernel's
    // 32-bit reach: 2 * (m + 1) * (2 * D) <= 2^32
    const long max_row = 0x80000000L / (2L * D) - 1;
    std::vector<kvp::gd::Sub> subs;
    for (long j = key_begin; j < key_end;) {
        const long m = map[j];
        if (m < 0 || m > max_row) {
            ++j;
            continue;
        }
        long r = 1;
        while (j + r < key_end && map[j + r] == m + r && m + r <= max_row &&
               (j + r - key_begin) % 16 != 0)
            ++r;
        kvp::gd::add_rows(subs, j, r, m, key_begin, key_end);
        j += r;
    }
    std::vector<kvp::gd::Ent> ents;
    kvp::gd::encode(subs, ents);
    std::fill(out, out + 2 * n, 0u);
    for (const kvp::gd::Ent& e : ents) {
        out[2 * e.g] = e.w0;
        out[2 * e.g + 1] = e.w1;
    }
    return n;
}

}  // extern "C"

// C++-linkage reference signatures (reference: src/attn_kernel.h:15-29).
void attn_forward_launcher(const float* d_q, const float* d_k, const float* d_v,
                           const float* d_arena, const long* d_kvmap, float* d_out,
                           int frames, int T, int D, int heads, bool remap) {
    (void)kvp_attn_forward_launcher(d_q, d_k, d_v, d_arena, d_kvmap, d_out, frames, T, D,
                                    heads, remap ? 1 : 0);
}

void attn_forward_single_frame(const float* d_q_f, const float* d_k, const float* d_v,
                               const float* d_arena, const long* d_kvmap_f, float* d_out_f,
                               int T, int D, int heads, int cross, int frame_idx) {
    (void)kvp_attn_forward_single_frame(d_q_f, d_k, d_v, d_arena, d_kvmap_f, d_out_f, T, D,
                                        heads, cross, frame_idx);
}
