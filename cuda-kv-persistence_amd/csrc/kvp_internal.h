#pragma once
// Internal helpers shared by the HIP translation units and the host C++ of
// libkvpersist.so. Not installed; the public surface is include/*.h.

#include <cstddef>

#include "kvp_c_api.h"

namespace kvp {

// Record a failure for kvp_last_error() (thread-local text).
void set_error(const char* fmt, ...);
void clear_error();

// Library stream for the reference-signature attention entry points.
void* library_stream();

// One attention launch (attn_fwd.hip), frames i = 0..frames-1 of it:
//   queries  q + i*q_fstride, rows [0, nq); output out + i*q_fstride;
//   keys     [max(key_begin, e - max_span), e), e = key_end + i*kend_step,
//            rows indexed against k/v + i*kv_fstride elements;
//   KVMap    kvmap + i*map_fstride entries, indexed by key row;
//   arena    arena + i*arena_fstride bytes (0: all frames share one arena).
// layer = true runs the whole set as one grid in the longest-first XCD
// column order with no key split (kend_step may then be non-zero; it must be
// 0 otherwise). max_span <= 0 means no limit. Split partials go to
// `workspace` when it is given (no allocation; at least
// attention_workspace_bytes(L) bytes), else to the library's per-(device,
// stream) buffer.
struct AttnLaunch {
    int dtype = 0;  // 0 = fp32, 1 = bf16
    const void* q = nullptr;
    const void* k = nullptr;
    const void* v = nullptr;
    const void* arena = nullptr;
    const long* kvmap = nullptr;
    // bf16 KVMap launches: optional group descriptors of the map (format:
    // kvp_attn_forward_frames_gd), gd_fstride entries per frame
    const unsigned* gdesc = nullptr;
    long gd_fstride = 0;
    void* out = nullptr;
    int nq = 0, D = 0, heads = 0, frames = 1;
    long q_fstride = 0, kv_fstride = 0, map_fstride = 0, arena_fstride = 0;
    long key_begin = 0, key_end = 0, kend_step = 0, max_span = 0;
    bool layer = false;
    bool cold_rows_nt = false;  // bf16 KVMap launches: original rows loaded non-temporally
    void* stream = nullptr;
    void* workspace = nullptr;
    size_t workspace_bytes = 0;
};
int launch_attention(const AttnLaunch& L);
// launch_attention with the split partials in the library's fixed device
// scratch array (64 MiB per GPU) instead of an allocated workspace; refuses
// launches whose partials exceed it. Allocates nothing.
int launch_attention_noalloc(AttnLaunch L);
// Split-partial bytes launch_attention(L) needs (0 when it does not split).
size_t attention_workspace_bytes(const AttnLaunch& L);

// Core attention launch (attn_fwd.hip). Queries q[frame*q_fstride + row*D]
// for rows [0, nq) of `frames` frames; keys [key_begin, key_end) against
// k/v bases offset by frame*kv_fstride elements and kvmap offset by
// frame*map_fstride entries. dtype 0 = fp32, 1 = bf16. Returns 0 on success.
int launch_attention(int dtype, const void* q, const void* k, const void* v,
                     const void* arena, const long* kvmap, void* out, int nq,
                     int D, int heads, int frames, long q_fstride,
                     long kv_fstride, long map_fstride, long key_begin,
                     long key_end, void* stream);

int attention_splits(int dtype, int nq, int heads, int frames, long span);

// Staging plans (kv_stage.hip): a flush with the arguments of kvp_stage_run,
// prepared without launching; stage_plan_launch launches it.
void* stage_plan_create(void* stager, void* arena, long row_stride_bytes,
                        const KvpRowCopy* copies, long n_copies, long* map_dev,
                        long map_fill, const long* map_rows,
                        const long* map_slots, long n_map);
int stage_plan_launch(const void* plan, void* stream);
void stage_plan_free(void* plan);

// Layer staging (kv_stage.hip): one launch that copies runs of consecutive
// K/V rows into consecutive arena rows ([K row | V row] per arena row) and
// writes runs of KVMap entries. Run tables travel through the stager's
// mapped descriptor ring.
constexpr int kLayerCopyRows = 32;     // rows per copy run (one workgroup)
constexpr int kLayerMapEntries = 1024; // entries per map run (one workgroup)
struct LayerCopyRun {
    int src_row;  // first K/V row (index into k and v, row_bytes apart)
    int dst_row;  // first arena row
    int n;        // rows, 1..kLayerCopyRows
    int pad;
};
struct LayerMapRun {
    long index;   // first KVMap entry
    int value;    // -1: n entries reset to -1; else entry j = value + j
    int n;        // entries, 1..kLayerMapEntries
};
// One entry of a group-descriptor table (2 words per entry).
struct LayerGdWrite {
    long index;   // entry index
    unsigned w0, w1;
};
// The caller has checked every run against its buffers: src rows below
// the K/V row count, dst rows below the arena's, map entries below the map's,
// descriptor entries below the table's.
// row_bytes: bytes of one K (or V) row, a multiple of 16.
int layer_stage_launch(void* stager, void* arena, const void* k, const void* v, long row_bytes,
                       const LayerCopyRun* copies, long n_copies, long* map,
                       const LayerMapRun* map_runs, long n_map_runs, unsigned* gd,
                       const LayerGdWrite* gd_writes, long n_gd_writes, void* stream);
// n 32-bit words at dst set to value, on the stream (a kernel, no memset node).
int fill_words(void* dst, long n, unsigned value, void* stream);

// Grouped bf16 projection GEMM (proj_gemm.hip): for g < groups (1..3),
// outs[g][r, n] = sum_k x[r, k] w[g*Ng + n, k] + bias[g*Ng + n]
// (+ outs[g][r, n] when accumulate; fp32 output only). x, w bf16; bias fp32
// or null; out_dtype 0 = fp32, 1 = bf16; tile_n 128 (128 x 128 tiles, two
// workgroups per CU) or 256 (256 x 256 tiles, one workgroup per CU).
// Returns 0 on success, 2 when the shape is outside the
// kernel's tiling (K % 64 or Ng % tile_n), 1 on any other error.
int launch_proj_gemm(const void* x, const void* w, const float* bias, void* const* outs,
                     int groups, long rows, int K, int Ng, int out_dtype, bool accumulate,
                     int tile_n, void* stream);
// Any-shape linear layer (proj_gemm.hip, fp32 matrix cores):
// y[r, n] = sum_k x[r, k] w[n, k] + bias[n] (+ y[r, n] when accumulate, fp32
// output only); in/out dtype pairs fp32->fp32, bf16->bf16, bf16->fp32.
int launch_gemm_generic(int in_dtype, int out_dtype, const void* x, const void* w,
                        const float* bias, void* y, long rows, int K, int N, bool accumulate,
                        void* stream);

}  // namespace kvp
