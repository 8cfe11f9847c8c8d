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

#include <algorithm>
#include <climits>
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

// Row id -> arena slot table of the streaming mode: open addressing with
// linear probing over a power-of-two array; erased entries leave tombstones
// that later inserts reuse, and the table is rebuilt when entries plus
// tombstones pass half of it. Keys kEmpty and kTomb mark free entries, so
// any row id but the two smallest longs can be stored. An implementation
// detail of KVTileManager, kept here because the class holds one.
class KvtmRowTable {
public:
    static constexpr long kEmpty = LONG_MIN;
    static constexpr long kTomb = LONG_MIN + 1;
    // Slot of row, or -1 when absent (slots are >= 0).
    long find(long row) const {
        if (keys_.empty()) return -1;
        for (size_t i = home(row);; i = (i + 1) & mask_) {
            if (keys_[i] == row) return vals_[i];
            if (keys_[i] == kEmpty) return -1;
        }
    }
    void insert(long row, long slot) {  // row must be absent
        if ((size_ + tombs_ + 1) * 2 > keys_.size()) rebuild();
        size_t i = home(row);
        while (keys_[i] != kEmpty && keys_[i] != kTomb) i = (i + 1) & mask_;
        if (keys_[i] == kTomb) --tombs_;
        keys_[i] = row;
        vals_[i] = slot;
        ++size_;
    }
    // Removes row; returns its slot, or -1 when absent.
    long erase(long row) {
        if (keys_.empty()) return -1;
        for (size_t i = home(row);; i = (i + 1) & mask_) {
            if (keys_[i] == row) {
                keys_[i] = kTomb;
                --size_;
                ++tombs_;
                return vals_[i];
            }
            if (keys_[i] == kEmpty) return -1;
        }
    }
    void clear() {
        std::fill(keys_.begin(), keys_.end(), kEmpty);
        size_ = 0;
        tombs_ = 0;
    }
    void reserve(size_t n) {
        if ((n + tombs_) * 2 > keys_.size()) rebuild(n);
    }
    size_t size() const { return size_; }

private:
    // Row ids are mostly dense (frame * T + token): consecutive ids take
    // consecutive buckets, so a tile's rows probe one or two cache lines;
    // the folded high bits break up ids that differ by a power of two.
    size_t home(long row) const {
        const unsigned long long r = (unsigned long long)row;
        return (size_t)(r ^ (r >> 17) ^ (r >> 34)) & mask_;
    }
    // Re-inserts the live entries into a table with room for at least
    // `want` of them at half load (tombstones dropped).
    void rebuild(size_t want = 0) {
        size_t cap = 64;
        while (cap < 4 * (size_ + 1) || cap < 2 * want) cap *= 2;
        std::vector<long> ok, ov;
        ok.swap(keys_);
        ov.swap(vals_);
        keys_.assign(cap, kEmpty);
        vals_.assign(cap, 0);
        mask_ = cap - 1;
        size_ = 0;
        tombs_ = 0;
        for (size_t i = 0; i < ok.size(); ++i)
            if (ok[i] != kEmpty && ok[i] != kTomb) insert(ok[i], ov[i]);
    }
    std::vector<long> keys_, vals_;
    size_t mask_ = 0;
    size_t size_ = 0;
    size_t tombs_ = 0;
};

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
    // Batched staging of n consecutive rows, row i's K at k_first + i*k_bytes
    // and V at v_first + i*v_bytes (null bases stay null): the decisions and
    // state of n calls of arena_stage, or of streaming_stage with row ids
    // row_first + i and changed = false, made in row order and stopped at the
    // first refusal. Returns the rows staged; their slots go to out_slots
    // when it is non-null. *copied receives the staged rows that needed a
    // copy (every row in arena mode; no sticky hits in streaming mode).
    long arena_stage_rows(const char* k_first, size_t k_bytes, const char* v_first,
                          size_t v_bytes, long n, long* out_slots);
    long streaming_stage_rows(long row_first, const char* k_first, size_t k_bytes,
                              const char* v_first, size_t v_bytes, long n,
                              long* out_slots, long* copied);

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

    KvtmRowTable row_slot_;
    std::vector<long> free_slots_;
    long slot_high_water_;
    size_t staged_bytes_;

    void* stream_;
    void* stager_;  // device-layer staging ring (kvp_stager_*)
    mutable std::vector<KvpRowCopy> pending_;
    mutable std::unordered_map<long, size_t> pending_by_row_;
};
