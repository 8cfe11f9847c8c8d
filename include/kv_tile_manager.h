#pragma once

// KVTileManager: budget accounting and the hot KV arena that feeds the
// KVMap-indirected attention kernel (attn_kernel.h).
//
// Public interface kept from the reference (reference:
// src/kv_tile_manager.h:15-66; semantics src/kv_tile_manager.cu:12-219):
//   * window mode  : admit / release / clear with exact byte accounting;
//   * arena mode   : per-step compaction of staged K|V rows into one
//                    contiguous arena, rows handed out sequentially;
//   * streaming    : sticky slots keyed by logical row id, LIFO free list,
//                    copy only on first admission or when content changed.
//
// MI355X re-derivation. CDNA4 has no persisting-L2 access-policy window, so
// init()/apply_window() do not program cache hardware. The budget is a
// residency budget: the arena is one contiguous allocation sized by the
// caller against gfx950's 4 MB per-XCD L2 / 256 MB Infinity Cache, and its
// residency is measured with TCC counters rather than requested. init()
// refuses budgets above the Infinity Cache (kvtm residency limit) the way the
// reference refused a carve-out above the device maximum.
//
// Staging copies are not issued one row at a time. Every stage call records
// a row copy; the pending copies of a step are executed by ONE gather kernel
// at the next flush point: arena_apply_window(), streaming_apply_window(),
// arena_device_ptr(), arena_begin_step(), arena_end_step(), streaming_end()
// or flush(). Source rows must not be modified by the caller between the
// stage call and that flush point. Copies run on the manager's stream
// (default: the null stream, as in the reference).
//
// Not thread-safe (same as the reference).

#include <cstddef>
#include <unordered_map>
#include <vector>

#include "kvp_c_api.h"

enum KvtmResult {
    KVTM_ADMITTED = 1,
    KVTM_REFUSED_BUDGET = 0,
    KVTM_INVALID = -1,  // bad args, duplicate admit
};

// Residency ceiling used by init(): gfx950 Infinity Cache (256 MiB).
static const size_t KVTM_RESIDENCY_LIMIT_BYTES = (size_t)256 << 20;

class KVTileManager {
public:
    KVTileManager(size_t budget_bytes, size_t max_window_bytes);
    ~KVTileManager();

    bool init();

    KvtmResult admit(long tile_id, void* ptr, size_t bytes);
    bool release(long tile_id);
    void clear();

    size_t persisted_bytes() const { return used_bytes_; }
    int persisted_tiles() const;
    bool is_persisted(long tile_id) const;
    size_t query_device_limit() const;

    // ---- arena mode ----
    bool arena_init(size_t capacity_bytes, size_t row_stride_floats);
    void arena_begin_step();
    bool arena_stage(const void* k_dev, size_t k_bytes, const void* v_dev,
                     size_t v_bytes, long* out_row);
    bool arena_apply_window();
    void arena_end_step();
    size_t arena_used_bytes() const { return arena_used_; }
    void* arena_device_ptr() const;

    // ---- streaming mode ----
    bool streaming_begin();
    bool streaming_stage(long row_id, const void* k_dev, size_t k_bytes,
                         const void* v_dev, size_t v_bytes, bool changed,
                         long* out_slot, bool* restaged);
    bool streaming_release(long row_id);
    bool streaming_apply_window();
    void streaming_end();
    size_t streaming_staged_bytes() const { return staged_bytes_; }

    // ---- additive (no reference counterpart) ----
    // Use caller-owned device memory as the arena (never freed here).
    // dev_ptr == nullptr gives a plan-only manager: all bookkeeping runs,
    // no copy is ever issued (used to compute KVMaps/slots on a host).
    bool arena_attach(void* dev_ptr, size_t capacity_bytes,
                      size_t row_stride_floats);
    // Execute pending staging copies now. false if a copy failed.
    bool flush() const;
    // Stream (hipStream_t) used for staging copies; nullptr = null stream.
    void set_stream(void* stream) { stream_ = stream; }
    void* stream() const { return stream_; }
    size_t arena_capacity_bytes() const { return arena_cap_; }
    size_t arena_row_stride_bytes() const {
        return arena_row_stride_floats_ * sizeof(float);
    }
    long streaming_capacity_rows() const;
    long streaming_high_water() const { return slot_high_water_; }
    size_t pending_copies() const { return pending_.size(); }
    // Flush pending copies and rebuild a device KVMap in the same launch
    // pair: map_dev[0..map_fill) = -1, then map_dev[map_rows[i]] =
    // map_slots[i]. Used by the frame pipeline (kvp_pipeline_*), which
    // builds the map on the device instead of uploading a host copy.
    bool flush_with_map(long* map_dev, long map_fill, const long* map_rows,
                        const long* map_slots, size_t n_map) const;
    // Same flush, prepared but not launched: *plan receives a staging plan
    // (launched later by the library, e.g. together with the attention
    // launch that precedes it; nullptr when there is nothing to do or the
    // manager is plan-only). The pending copies are handed over at once.
    bool flush_plan(void** plan, long* map_dev, long map_fill, const long* map_rows,
                    const long* map_slots, size_t n_map) const;

private:
    bool record_copy(long dst_row, const void* k_dev, size_t k_bytes,
                     const void* v_dev, size_t v_bytes);
    bool row_fits(long row, size_t total) const;

    struct Entry {
        void* ptr;
        size_t bytes;
    };

    std::unordered_map<long, Entry> active_;
    size_t budget_bytes_;
    size_t max_window_bytes_;
    size_t used_bytes_;
    bool initialized_;
    size_t device_limit_;

    void* arena_;
    bool arena_owned_;
    bool plan_only_;
    size_t arena_cap_;
    size_t arena_row_stride_floats_;
    size_t arena_next_row_;
    size_t arena_used_;

    std::unordered_map<long, long> row_slot_;
    std::vector<long> free_slots_;
    long slot_high_water_;
    size_t staged_bytes_;

    void* stream_;
    void* stager_;  // device-layer staging ring (kvp_stager_*)
    mutable std::vector<KvpRowCopy> pending_;
    mutable std::unordered_map<long, size_t> pending_by_row_;
};
