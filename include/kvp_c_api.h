#pragma once

/*
 * C-ABI of libkvpersist.so: the drop-in boundary for the reference's
 * KVMap-indirected attention + KV-arena hot path, MI355X (gfx950) native.
 *
 * Conventions
 *   - `long` is LP64 int64, as in the reference facade.
 *   - Every pointer named d_* / *_dev / q,k,v,out,arena,kvmap is a device
 *     pointer owned by the caller unless stated otherwise.
 *   - Entry points returning int report 0 = success (attention, device and
 *     pipeline layers) unless they mirror a reference function, in which case
 *     they keep the reference's return convention (noted per block).
 *   - kvp_last_error() holds the text of the most recent failure.
 *   - Layout: token-major [rows, D], D = heads * 128, element (t, h, d) at
 *     t*D + h*128 + d. Arena row = [K row (D) | V row (D)], stride 2*D
 *     elements. KVMap[j] >= 0 -> key row j lives at arena row KVMap[j];
 *     KVMap[j] < 0 -> read the original K/V row j. The bf16 kernels address
 *     the arena with 32-bit byte offsets: an entry m counts only while
 *     2*(m+1)*row_bytes <= 2^32 (its row lies in the arena's first 4 GiB);
 *     a larger entry reads the original row as a negative one does.
 */

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------
 * KVTileManager facade. Same symbols, signatures and return conventions as
 * the reference ctypes contract (reference: src/kv_tile_manager.cu:223-341):
 * ints are 1 = ok / 0 = refused, kvtm_admit returns 1 / 0 / -1.
 * ---------------------------------------------------------------------- */
void* kvtm_create(long budget_bytes, long max_window_bytes);      /* cu:225 */
void kvtm_destroy(void* m);                                       /* cu:234 */
int kvtm_init(void* m);                                           /* cu:236 */
long kvtm_query_limit(void* m);                                   /* cu:240 */
int kvtm_admit(void* m, long tile_id, void* ptr, long bytes);     /* cu:244 */
int kvtm_release(void* m, long tile_id);                          /* cu:249 */
void kvtm_clear(void* m);                                         /* cu:253 */
long kvtm_persisted_bytes(void* m);                               /* cu:255 */
int kvtm_persisted_tiles(void* m);                                /* cu:259 */
void* kvtm_dev_alloc(long bytes);                                 /* cu:264 */
void kvtm_dev_free(void* p);                                      /* cu:270 */
int kvtm_arena_init(void* m, long cap_bytes, long row_stride_floats); /* cu:274 */
void kvtm_arena_begin(void* m);                                   /* cu:280 */
int kvtm_arena_stage(void* m, const void* k_dev, long k_bytes,
                     const void* v_dev, long v_bytes, long* out_row); /* cu:281 */
int kvtm_arena_window(void* m);                                   /* cu:289 */
void kvtm_arena_end(void* m);                                     /* cu:292 */
long kvtm_arena_used(void* m);                                    /* cu:293 */
void* kvtm_arena_ptr(void* m);                                    /* cu:296 */
int kvtm_streaming_begin(void* m);                                /* cu:302 */
int kvtm_streaming_stage(void* m, long row_id, const void* k_dev,
                         long k_bytes, const void* v_dev, long v_bytes,
                         int changed, long* out_slot, int* restaged); /* cu:305 */
int kvtm_streaming_release(void* m, long row_id);                 /* cu:317 */
int kvtm_streaming_window(void* m);                               /* cu:320 */
void kvtm_streaming_end(void* m);                                 /* cu:323 */
long kvtm_streaming_staged_bytes(void* m);                        /* cu:326 */
long kvtm_layout_tiles_per_frame(int tokens_per_frame, int tile_tokens); /* cu:331 */
long kvtm_layout_tile_start(int tpf, int tt, long id);            /* cu:334 */
int kvtm_layout_tile_count(int tpf, int tt, long id);             /* cu:337 */

/* Additive manager entry points (no reference counterpart). */
/* Caller-owned arena; dev_ptr NULL = plan-only manager (no device copies). */
int kvtm_arena_attach(void* m, void* dev_ptr, long cap_bytes,
                      long row_stride_floats);
int kvtm_flush(void* m);                      /* 1 = ok */
void kvtm_set_stream(void* m, void* stream);  /* hipStream_t, NULL = null stream */
int kvtm_is_persisted(void* m, long tile_id); /* reference: kv_tile_manager.h:35 */
long kvtm_streaming_high_water(void* m);
long kvtm_streaming_capacity(void* m);
long kvtm_pending_copies(void* m);

/* ------------------------------------------------------------------------
 * Tile gating policies (reference: src/tile_gating_policy.h:8-68).
 * ---------------------------------------------------------------------- */
/* name: "none" | "uniform" | "recency" | "motion" | "reuse_weighted";
 * NULL for an unknown name. */
void* kvp_policy_create(const char* name, int tiles_per_frame,
                        int total_frames);
void kvp_policy_destroy(void* p);
const char* kvp_policy_name(void* p);
/* TileGatingPolicy::select; returns the count written to out_ids
 * (out_ids must hold max_tiles entries). */
int kvp_policy_select(void* p, const float* scores, int num_candidates,
                      int max_tiles, long* out_ids);
/* TileGatingPolicy::select_range (window-aware, ids absolute). */
int kvp_policy_select_range(void* p, const float* scores_flat, long first_id,
                            int num_candidates, int max_tiles, long* out_ids);

/* ------------------------------------------------------------------------
 * Attention. FP32 entry points mirror the reference C++ functions
 * (reference: src/attn_kernel.h:15-29, src/gated_attention_kernel.cu:141-184)
 * argument for argument; they return 0 on success (the C++ wrappers in
 * attn_kernel.h drop the code, as the reference's void functions do).
 * head_dim must be 128 (D == heads * 128), as in the reference kernel.
 * Launches go to the library stream set by kvp_set_stream (default: null
 * stream, as in the reference).
 * ---------------------------------------------------------------------- */
int kvp_attn_forward_launcher(const float* d_q, const float* d_k,
                              const float* d_v, const float* d_arena,
                              const long* d_kvmap, float* d_out, int frames,
                              int T, int D, int heads, int remap);
int kvp_attn_forward_single_frame(const float* d_q_f, const float* d_k,
                                  const float* d_v, const float* d_arena,
                                  const long* d_kvmap_f, float* d_out_f,
                                  int T, int D, int heads, int cross,
                                  int frame_idx);

/* bf16 storage (raw uint16 bit patterns), fp32 accumulation, bf16 output.
 * Additive: the reference is fp32-only. */
int kvp_attn_forward_launcher_bf16(const void* d_q, const void* d_k,
                                   const void* d_v, const void* d_arena,
                                   const long* d_kvmap, void* d_out,
                                   int frames, int T, int D, int heads,
                                   int remap);
/* window_frames = 0: causal prefix [0, (frame_idx+1)*T) as the reference;
 * window_frames = W > 0: sliding window [max(0, f-W+1)*T, (f+1)*T).
 * Ignored when cross == 0. */
int kvp_attn_forward_single_frame_bf16(const void* d_q_f, const void* d_k,
                                       const void* d_v, const void* d_arena,
                                       const long* d_kvmap_f, void* d_out_f,
                                       int T, int D, int heads, int cross,
                                       int frame_idx, int window_frames);
int kvp_attn_forward_single_frame_window(const float* d_q_f, const float* d_k,
                                         const float* d_v,
                                         const float* d_arena,
                                         const long* d_kvmap_f, float* d_out_f,
                                         int T, int D, int heads, int cross,
                                         int frame_idx, int window_frames);

/* General form: queries q[0..nq) (pre-offset), keys [key_begin, key_end)
 * indexed against k/v/kvmap bases. dtype 0 = fp32, 1 = bf16. */
int kvp_attn_forward_range(int dtype, const void* q, const void* k,
                           const void* v, const void* arena,
                           const long* kvmap, void* out, int nq, int D,
                           int heads, long key_begin, long key_end,
                           void* stream);

/* Allocation-free form of kvp_attn_forward_range, same arguments and
 * results bit for bit. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc). It calls no hipMalloc,
 * hipFree or allocating library routine: the split partials of the launch
 * live in a fixed 64 MiB device array of the library (one per GPU, held
 * until the process ends), and a launch whose partials exceed it returns 1
 * with the reason in kvp_last_error(). All calls on one GPU share that array:
 * calls that overlap on one GPU (other streams, other threads) race. */
int kvp_attn_forward_range_noalloc(int dtype, const void* q, const void* k,
                                   const void* v, const void* arena,
                                   const long* kvmap, void* out, int nq, int D,
                                   int heads, long key_begin, long key_end,
                                   void* stream);

/* A whole layer in one launch (additive; the reference launches one frame
 * at a time). q/out: [frames*T, D]; k/v: [frames*T, D] (absolute rows).
 * Frame f's queries q[f*T .. (f+1)*T) attend
 *   cross == 0: the keys of frame f, KVMap slice kvmap + f*map_frame_stride
 *               indexed by frame-relative key (the reference's remap slice);
 *   cross != 0: keys [max(0, f+1-W)*T, (f+1)*T) (W = window_frames, 0 = the
 *               whole causal prefix), slice kvmap + f*map_frame_stride indexed
 *               by absolute key row.
 * Frame f's arena is arena + f*arena_frame_bytes (0: one shared arena). The
 * frames run as one grid, longest key range first, with no key split.
 * flags: KVP_ATTN_COLD_ROWS_NT = with a KVMap (bf16), rows read from the
 * original K/V buffers are loaded non-temporally, so the L2 evicts them
 * before arena lines. An additive CDNA4 residency lever with no
 * counterpart in the reference: its persisting window (hitRatio 1,
 * src/kv_tile_manager.cu:39-47) streams no access, and rows outside the
 * window are cached normally there. */
#define KVP_ATTN_COLD_ROWS_NT 1
int kvp_attn_forward_frames(int dtype, const void* q, const void* k,
                            const void* v, const void* arena,
                            long arena_frame_bytes, const long* kvmap,
                            long map_frame_stride, void* out, int frames,
                            int T, int D, int heads, int cross,
                            int window_frames, int flags, void* stream);

/* kvp_attn_forward_frames for bf16 KVMap launches with group descriptors
 * (additive; no counterpart in the reference). gdesc: per frame,
 * gd_frame_stride entries of two 32-bit words, frame f's table at
 * gdesc + 2*f*gd_frame_stride. Entry g describes rows [b + 16g, b + 16g + 16)
 * of frame f's key range [b, e) (rows at or past e excluded), the copy
 * group of one wave of the bf16 kernel; gd_frame_stride must cover
 * 4 * ceil(longest range / 64) entries. Entry (w0, w1):
 *   w0 == 0     no row of the group is read from the arena;
 *   w0 == 1     general: the kernel reads the group's KVMap entries;
 *   w0 bit 31   sub-run: rows r0 .. r0+n-1 of the group map to arena rows
 *               l .. l+n-1 (l = bits 0-22, r0 = bits 23-26, n-1 = bits
 *               27-30); w1 is a second sub-run word or 0; every other row
 *               of the group maps to no arena row.
 * The table must describe the map exactly (kvp_attn_group_desc builds it
 * from a host copy of a map slice). With it the kernel reads a group's map
 * entries only for general groups; outputs are bitwise those of
 * kvp_attn_forward_frames with the same map. */
int kvp_attn_forward_frames_gd(const void* q, const void* k, const void* v,
                               const void* arena, long arena_frame_bytes,
                               const long* kvmap, long map_frame_stride,
                               const unsigned* gdesc, long gd_frame_stride,
                               void* out, int frames, int T, int D, int heads,
                               int cross, int window_frames, void* stream);
/* Host builder of one frame's descriptor table: map[j] is the KVMap entry
 * of key j (the slice the frame reads), [key_begin, key_end) the frame's key
 * range, D the hidden size (an entry m counts as an arena row when
 * 0 <= m and 2*(m+1)*2*D <= 2^32, as in the bf16 kernel). Writes the
 * 4*ceil((key_end-key_begin)/64) entries (2 words each) to out when cap
 * (in entries) holds them; returns the entry count, or -1 on bad
 * arguments. */
long kvp_attn_group_desc(const long* map, long key_begin, long key_end, int D,
                         unsigned* out, long cap);

/* Split-partial workspaces (per-frame launches that split their key range
 * keep one device buffer per (device, stream), per thread for
 * hipStreamPerThread; at most 8 per device, least recently used freed
 * first). kvp_attn_workspace_release frees the calling device's buffer of
 * `stream` after synchronising it (0 on success); kvp_attn_workspace_count
 * is the number of buffers held on all devices. No reference counterpart. */
int kvp_attn_workspace_release(void* stream);
long kvp_attn_workspace_count(void);

void kvp_set_stream(void* stream);
void* kvp_get_stream(void);
const char* kvp_last_error(void);
int kvp_device_count(void);

/* Attention kernel constants exported for callers (reference:
 * src/attn_kernel.h:31-32 exports its tile shape the same way). */
int kvp_attn_block_queries(int dtype);
int kvp_attn_block_keys(int dtype);
/* Split count chosen for a launch of nq queries x heads x frames over
 * span keys (key-split flash decoding when the grid would underfill). */
int kvp_attn_splits(int dtype, int nq, int heads, int frames, long span);

/* ------------------------------------------------------------------------
 * Device layer used by the host C++ (manager / pipeline).
 * ---------------------------------------------------------------------- */
typedef struct KvpRowCopy {
    const void* k_src;     /* device address of the K row            */
    const void* v_src;     /* device address of the V row            */
    long dst_row;          /* arena row; K at row*stride, V after it */
    unsigned int k_bytes;
    unsigned int v_bytes;
} KvpRowCopy;

void* kvp_dev_alloc(size_t bytes);
void kvp_dev_free(void* p);
int kvp_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int kvp_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int kvp_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int kvp_stream_sync(void* stream);
int kvp_device_sync(void);

/* Staging ring: mapped coherent host memory holding the launches' run
 * descriptors, reused across flushes; when it wraps it first waits for the
 * launches that read it (destroying a stager waits for the device). */
void* kvp_stager_create(void);
void kvp_stager_destroy(void* stager);
/* One flush: optional map rebuild (map_dev[0..map_fill) = -1 then
 * map_dev[map_rows[i]] = map_slots[i]) followed by one gather kernel that
 * performs every row copy. Returns 0 on success. */
int kvp_stage_run(void* stager, void* arena, long row_stride_bytes,
                  const KvpRowCopy* copies, long n_copies, long* map_dev,
                  long map_fill, const long* map_rows, const long* map_slots,
                  long n_map, void* stream);

/* ------------------------------------------------------------------------
 * Frame pipeline: the per-frame select -> release -> stage -> map ->
 * attention loop of the reference driver
 * (reference: src/run_policy_experiment.cu:136-283), as a library object.
 * ---------------------------------------------------------------------- */
/* dtype 0 = fp32, 1 = bf16. cross 0/1 = intra / causal cross-frame.
 * window_frames 0 = full prefix. plan_only 1 = bookkeeping only (no device
 * work; attention is not run). Returns NULL on bad arguments. */
void* kvp_pipeline_create(const char* policy, int cross, int streaming,
                          int frames, int T, int D, int heads,
                          int tile_tokens, long set_aside_bytes, int dtype,
                          int window_frames, int plan_only);
void kvp_pipeline_destroy(void* p);
int kvp_pipeline_set_stream(void* p, void* stream);
/* Residency lever of the pipeline's attention launches: 1 = original K/V
 * rows non-temporal (KVP_ATTN_COLD_ROWS_NT), 0 = default. */
int kvp_pipeline_set_cold_rows_nt(void* p, int on);
/* Run frame f (frames must be stepped in order 0,1,...). q/k/v/out are the
 * full [frames*T, D] buffers; scores_flat is [frames][tiles_per_frame]
 * (may be NULL for policy none). Returns 0 on success. */
int kvp_pipeline_step(void* p, int f, const void* q, const void* k,
                      const void* v, void* out, const float* scores_flat);
/* A whole layer, frames 0..frames-1 (streaming state is reset first), in
 * two launches: every frame's host plan is made first, then one staging
 * launch copies the rows the frames map into a layer arena and writes frame
 * f's KVMap to slice f of a layer map, pointing each row frame f maps at its
 * physical row (and, in bf16, the group descriptors of every slice, see
 * kvp_attn_forward_frames_gd); then one attention launch runs all frames,
 * frame f reading its own slice. K and V are fixed for the layer, so one
 * copy of a row serves every frame that maps it: each tile some frame maps
 * gets physical rows for the longest prefix of it any frame maps, tiles in
 * key order. The layer arena is allocated once at frames x rows-per-set-
 * aside rows of [K | V] (the set-aside summed over the frames; no frame maps
 * more than the set-aside, so the run always fits). Each frame maps exactly
 * the rows frame-by-frame stepping maps: outputs are bitwise equal across
 * policies and modes within kvp_pipeline_run, and equal stepping's up to
 * the rounding of stepping's key split. The layer map holds frames slices
 * of frames*T (cross) or T (intra) entries, absolute key rows in cross mode,
 * frame-relative in intra mode. A plan-only pipeline makes the same plans
 * and applies the staging launch's runs to host copies of the map, the
 * descriptor tables and each physical row's source row, launching nothing
 * (kvp_pipeline_layer_plan_map / _plan_gd / _plan_sources). After a failed
 * run the layer state is rebuilt from scratch by the next run. */
int kvp_pipeline_run(void* p, const void* q, const void* k, const void* v,
                     void* out, const float* scores_flat);
/* Introspection of the last step. */
int kvp_pipeline_selected(void* p, long* ids, int cap);
long kvp_pipeline_map(void* p, long* out, long cap);
long kvp_pipeline_slots(void* p);
long kvp_pipeline_staged_tiles(void* p);
long kvp_pipeline_staged_bytes(void* p);
long kvp_pipeline_copy_rows(void* p);
/* Step mode's arena and device KVMap (kvp_pipeline_step). */
void* kvp_pipeline_arena(void* p);
const long* kvp_pipeline_device_map(void* p);
void* kvp_pipeline_manager(void* p);
/* Layer mode (kvp_pipeline_run): the arena every frame reads, slice f at
 * map + f*map_stride entries, and the rows the last run copied into the
 * arena; NULL / 0 before the first run. */
void* kvp_pipeline_layer_arena(void* p);
const long* kvp_pipeline_layer_map(void* p);
long kvp_pipeline_layer_map_stride(void* p);
long kvp_pipeline_layer_copied_rows(void* p);
/* Bytes allocated for the layer arena (0 before the first run). */
long kvp_pipeline_layer_arena_bytes(void* p);
/* Group descriptors of the layer map (bf16; NULL otherwise): frame f's
 * table at gd + 2*f*stride words. */
const unsigned* kvp_pipeline_layer_gd(void* p);
long kvp_pipeline_layer_gd_stride(void* p);
/* The attention launch of the last kvp_pipeline_run again (same arena, map
 * slices and descriptors), on the pipeline's stream: the kernel the run
 * timed alone. Returns 0 on success. */
int kvp_pipeline_layer_attention(void* p, const void* q, const void* k,
                                 const void* v, void* out);
/* Plan-only pipelines, after kvp_pipeline_run: slice f of the layer map
 * (returns map_stride, copies min(map_stride, cap) entries) and the K/V row
 * each physical row holds (returns the row count, copies min(count, cap));
 * -1 for pipelines that are not plan-only or before the first run. */
long kvp_pipeline_layer_plan_map(void* p, int f, long* out, long cap);
long kvp_pipeline_layer_plan_sources(void* p, long* out, long cap);
/* Plan-only: frame f's descriptor table (returns the stride in entries,
 * copies min(stride, cap) entries of 2 words); -1 as above. */
long kvp_pipeline_layer_plan_gd(void* p, int f, unsigned* out, long cap);

#ifdef __cplusplus
}
#endif
