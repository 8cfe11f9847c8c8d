// Run-encoded arena flush (libkvpersist.so internal, HIP translation units
// only): the argument-block format of a staging flush and the work of one
// of its workgroups. A flush whose row copies form few runs (consecutive
// sources to consecutive arena rows) and whose KVMap updates form few runs
// (consecutive rows with consecutive slots, or resets to -1) travels as a
// kernel argument block; reference semantics of the copies:
// src/kv_tile_manager.cu:104-121, :153-192.
#pragma once

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdint>

#include "kvp_c_api.h"

namespace kvp {
namespace stage {

// Workgroup size of every kernel that runs stage_runs_block.
constexpr int kRunThreads = 256;

// Run-encoded flush, passed by value as the kernel's argument block
// (kept under 2 KiB).
constexpr int kMaxCopyRuns = 24;
constexpr int kMaxMapRuns = 64;

struct CopyRun {
    const unsigned char* k;  // K source of the run's first row
    const unsigned char* v;  // V source of the run's first row
    long dst_row;            // arena row of the run's first row
};

struct RunArgs {
    unsigned char* arena;
    long row_stride;
    long* map;
    int k_bytes, v_bytes;  // per row, the same for every row of the flush
    int n_entries;
    int row_blocks;        // workgroups [0, row_blocks) copy rows
    int vec16;             // sources, arena and sizes 16-byte aligned
    int pad;
    // Index of each run's first row / entry; unused slots hold INT_MAX, so
    // the run of item x is (number of firsts <= x) - 1 over the whole table,
    // a count whose loads do not depend on one another.
    int copy_first[kMaxCopyRuns];
    int map_first[kMaxMapRuns];
    CopyRun copy[kMaxCopyRuns];
    long map_row[kMaxMapRuns];  // first KVMap row of each map run
    int map_slot[kMaxMapRuns];  // slot of that row; -1 for a run of resets
};
static_assert(sizeof(RunArgs) <= 2048, "run-encoded flush must stay a small argument block");

// Work of workgroup b of a run-encoded flush (256 threads): b <
// row_blocks copies one row, the workgroups after that apply 256 map
// entries each. Used by the staging kernel and, as trailing workgroups, by
// the split-combine kernel of the attention launch that precedes the flush.
__device__ __forceinline__ void stage_runs_block(const RunArgs& a, int b) {
    if (b < a.row_blocks) {
        int r = -1;
#pragma unroll
        for (int i = 0; i < kMaxCopyRuns; ++i) r += a.copy_first[i] <= b ? 1 : 0;
        const long j = b - a.copy_first[r];
        unsigned char* dst = a.arena + (a.copy[r].dst_row + j) * a.row_stride;
        const unsigned char* ks = a.copy[r].k + j * a.k_bytes;
        const unsigned char* vs = a.copy[r].v + j * a.v_bytes;
        if (a.vec16) {
            typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
            const unsigned nk = (unsigned)a.k_bytes >> 4;
            const unsigned n = nk + ((unsigned)a.v_bytes >> 4);
            for (unsigned i = threadIdx.x; i < n; i += 256) {
                const u32x4* src = i < nk ? reinterpret_cast<const u32x4*>(ks) + i
                                          : reinterpret_cast<const u32x4*>(vs) + (i - nk);
                reinterpret_cast<u32x4*>(dst)[i] = *src;
            }
        } else {
            const unsigned n = (unsigned)a.k_bytes + (unsigned)a.v_bytes;
            for (unsigned i = threadIdx.x; i < n; i += 256)
                dst[i] = i < (unsigned)a.k_bytes ? ks[i] : vs[i - a.k_bytes];
        }
    } else {
        const int e = (b - a.row_blocks) * 256 + (int)threadIdx.x;
        if (e >= a.n_entries) return;
        int r = -1;
#pragma unroll
        for (int i = 0; i < kMaxMapRuns; ++i) r += a.map_first[i] <= e ? 1 : 0;
        const long j = e - a.map_first[r];
        const int slot = a.map_slot[r];
        a.map[a.map_row[r] + j] = slot < 0 ? -1L : (long)slot + j;
    }
}

// Builds the run encoding of a flush; false when it does not fit (more runs
// than the argument block holds, mixed row sizes, counts or slots beyond int).
inline bool encode_runs(RunArgs& ra, unsigned char* arena, long row_stride, const KvpRowCopy* copies,
                 long n_copies, long* map, const long* map_rows, const long* map_slots,
                 long n_map) {
    if (n_copies > (1L << 30) || n_map > (1L << 30)) return false;
    ra.arena = arena;
    ra.row_stride = row_stride;
    ra.map = map;
    ra.n_entries = (int)n_map;
    ra.row_blocks = (int)n_copies;
    ra.pad = 0;
    ra.k_bytes = n_copies > 0 ? (int)copies[0].k_bytes : 0;
    ra.v_bytes = n_copies > 0 ? (int)copies[0].v_bytes : 0;
    for (int i = 0; i < kMaxCopyRuns; ++i) ra.copy_first[i] = INT_MAX;
    for (int i = 0; i < kMaxMapRuns; ++i) ra.map_first[i] = INT_MAX;
    uintptr_t align = (uintptr_t)arena | (uintptr_t)row_stride | (uintptr_t)ra.k_bytes |
                      (uintptr_t)ra.v_bytes;
    int nc = 0;
    for (long i = 0; i < n_copies; ++i) {
        const KvpRowCopy& c = copies[i];
        if ((int)c.k_bytes != ra.k_bytes || (int)c.v_bytes != ra.v_bytes) return false;
        align |= (uintptr_t)c.k_src | (uintptr_t)c.v_src;
        const unsigned char* k = static_cast<const unsigned char*>(c.k_src);
        const unsigned char* v = static_cast<const unsigned char*>(c.v_src);
        if (nc > 0) {
            const CopyRun& last = ra.copy[nc - 1];
            const long j = i - ra.copy_first[nc - 1];
            if (k == last.k + j * ra.k_bytes && v == last.v + j * ra.v_bytes &&
                c.dst_row == last.dst_row + j)
                continue;
        }
        if (nc == kMaxCopyRuns) return false;
        ra.copy[nc] = CopyRun{k, v, c.dst_row};
        ra.copy_first[nc++] = (int)i;
    }
    int nm = 0;
    for (long i = 0; i < n_map; ++i) {
        const long row = map_rows[i];
        const long slot = map_slots[i] < 0 ? -1L : map_slots[i];
        if (slot > 0x7fffffffL) return false;
        if (nm > 0) {
            const long j = i - ra.map_first[nm - 1];
            const long last_slot = ra.map_slot[nm - 1];
            if (row == ra.map_row[nm - 1] + j &&
                ((last_slot < 0 && slot < 0) || (last_slot >= 0 && slot == last_slot + j)))
                continue;
        }
        if (nm == kMaxMapRuns) return false;
        ra.map_row[nm] = row;
        ra.map_slot[nm] = (int)slot;
        ra.map_first[nm++] = (int)i;
    }
    ra.vec16 = (align & 15u) == 0;
    return true;
}

// Workgroups a run-encoded flush needs.
inline long run_blocks(const RunArgs& a) {
    return (long)a.row_blocks + (a.n_entries + kRunThreads - 1) / kRunThreads;
}

}  // namespace stage
}  // namespace kvp
