// KVTileManager host implementation (g++; device work only through the
// kvp_* C-ABI device layer). Accounting and slot semantics follow the
// reference (reference: src/kv_tile_manager.cu:12-219) so that staging
// decisions, arena row order and KVMap contents are bit-identical; the
// device side differs: copies are batched into one gather launch per flush
// and no L2 persistence state exists on CDNA4.

#include "kv_tile_manager.h"
#include "kvp_internal.h"

#include <algorithm>
#include <cstdint>
#include <cstdio>

KVTileManager::KVTileManager(size_t budget_bytes, size_t max_window_bytes)
    : budget_bytes_(budget_bytes), max_window_bytes_(max_window_bytes),
      used_bytes_(0), initialized_(false), device_limit_(0), arena_(nullptr),
      arena_owned_(false), plan_only_(false), arena_cap_(0),
      arena_row_stride_floats_(0), arena_next_row_(0), arena_used_(0),
      slot_high_water_(-1), staged_bytes_(0), stream_(nullptr),
      stager_(nullptr) {}

KVTileManager::~KVTileManager() {
    clear();
    // Pending copies still land (an attached arena outlives the manager);
    // then the descriptor ring waits for its launches before it is freed.
    flush();
    if (stager_) {
        kvp_stager_destroy(stager_);  // waits for the launches that read it
        stager_ = nullptr;
    }
    if (arena_ && arena_owned_) {
        kvp_stream_sync(stream_);
        kvp_dev_free(arena_);
    }
}

// The reference programs the persisting-L2 carve-out here
// (cudaDeviceSetLimit, src/kv_tile_manager.cu:23-31). CDNA4 has none; the
// budget becomes a residency budget checked against the Infinity Cache.
bool KVTileManager::init() {
    if (budget_bytes_ > KVTM_RESIDENCY_LIMIT_BYTES) return false;
    device_limit_ = budget_bytes_;
    initialized_ = true;
    return true;
}

size_t KVTileManager::query_device_limit() const { return device_limit_; }

// reference: src/kv_tile_manager.cu:49-60 (argument checks, duplicate,
// window size, then the budget gate).
KvtmResult KVTileManager::admit(long tile_id, void* ptr, size_t bytes) {
    if (!initialized_ || tile_id < 0 || ptr == nullptr || bytes == 0)
        return KVTM_INVALID;
    if (active_.count(tile_id)) return KVTM_INVALID;
    if (bytes > max_window_bytes_) return KVTM_INVALID;
    if (used_bytes_ + bytes > budget_bytes_) return KVTM_REFUSED_BUDGET;
    active_[tile_id] = Entry{ptr, bytes};
    used_bytes_ += bytes;
    return KVTM_ADMITTED;
}

bool KVTileManager::release(long tile_id) {
    auto it = active_.find(tile_id);
    if (it == active_.end()) return false;
    used_bytes_ -= it->second.bytes;
    active_.erase(it);
    return true;
}

void KVTileManager::clear() {
    if (active_.empty()) return;
    active_.clear();
    used_bytes_ = 0;
}

int KVTileManager::persisted_tiles() const { return (int)active_.size(); }

bool KVTileManager::is_persisted(long tile_id) const {
    return active_.count(tile_id) != 0;
}

// ---- arena mode (reference: src/kv_tile_manager.cu:88-137) ----

bool KVTileManager::arena_init(size_t capacity_bytes, size_t row_stride_floats) {
    if (arena_ || plan_only_) return false;
    if (capacity_bytes == 0 || row_stride_floats == 0) return false;
    void* p = kvp_dev_alloc(capacity_bytes);
    if (!p) return false;
    arena_ = p;
    arena_owned_ = true;
    arena_cap_ = capacity_bytes;
    arena_row_stride_floats_ = row_stride_floats;
    arena_next_row_ = 0;
    arena_used_ = 0;
    return true;
}

bool KVTileManager::arena_attach(void* dev_ptr, size_t capacity_bytes,
                                 size_t row_stride_floats) {
    if (arena_ || plan_only_) return false;
    if (capacity_bytes == 0 || row_stride_floats == 0) return false;
    arena_ = dev_ptr;
    arena_owned_ = false;
    plan_only_ = (dev_ptr == nullptr);
    arena_cap_ = capacity_bytes;
    arena_row_stride_floats_ = row_stride_floats;
    arena_next_row_ = 0;
    arena_used_ = 0;
    return true;
}

void KVTileManager::arena_begin_step() {
    flush();
    arena_next_row_ = 0;
    arena_used_ = 0;
}

bool KVTileManager::row_fits(long row, size_t total) const {
    if (row < 0) return false;
    const size_t stride = arena_row_stride_floats_ * sizeof(float);
    return (size_t)row * stride + total <= arena_cap_;
}

bool KVTileManager::record_copy(long dst_row, const void* k_dev, size_t k_bytes,
                                const void* v_dev, size_t v_bytes) {
    if (plan_only_) return true;
    if (k_bytes > 0xffffffffu || v_bytes > 0xffffffffu) return false;
    KvpRowCopy c;
    c.k_src = k_dev;
    c.v_src = v_dev;
    c.dst_row = dst_row;
    c.k_bytes = (unsigned)k_bytes;
    c.v_bytes = (unsigned)v_bytes;
    // A later copy to the same row supersedes an earlier unflushed one (no
    // device work read the row in between), which keeps one launch free of
    // write races.
    auto it = pending_by_row_.find(dst_row);
    if (it != pending_by_row_.end()) {
        pending_[it->second] = c;
    } else {
        pending_by_row_[dst_row] = pending_.size();
        pending_.push_back(c);
    }
    return true;
}

bool KVTileManager::flush() const {
    return flush_with_map(nullptr, 0, nullptr, nullptr, 0);
}

bool KVTileManager::flush_with_map(long* map_dev, long map_fill,
                                   const long* map_rows, const long* map_slots,
                                   size_t n_map) const {
    if (plan_only_) return true;
    if (pending_.empty() && !map_dev) return true;
    KVTileManager* self = const_cast<KVTileManager*>(this);
    if (!self->stager_) {
        self->stager_ = kvp_stager_create();
        if (!self->stager_) return false;
    }
    const int rc = kvp_stage_run(stager_, arena_,
                                 (long)(arena_row_stride_floats_ * sizeof(float)),
                                 pending_.data(), (long)pending_.size(), map_dev,
                                 map_fill, map_rows, map_slots, (long)n_map,
                                 stream_);
    pending_.clear();
    pending_by_row_.clear();
    return rc == 0;
}

bool KVTileManager::flush_plan(void** plan, long* map_dev, long map_fill, const long* map_rows,
                               const long* map_slots, size_t n_map) const {
    *plan = nullptr;
    if (plan_only_) return true;
    if (pending_.empty() && !map_dev) return true;
    KVTileManager* self = const_cast<KVTileManager*>(this);
    if (!self->stager_) {
        self->stager_ = kvp_stager_create();
        if (!self->stager_) return false;
    }
    *plan = kvp::stage_plan_create(stager_, arena_, (long)(arena_row_stride_floats_ * sizeof(float)),
                                   pending_.data(), (long)pending_.size(), map_dev, map_fill, map_rows,
                                   map_slots, (long)n_map);
    pending_.clear();
    pending_by_row_.clear();
    return *plan != nullptr;
}

// reference: src/kv_tile_manager.cu:104-121 — both gates use the running
// byte total; rows are handed out sequentially in staging order.
bool KVTileManager::arena_stage(const void* k_dev, size_t k_bytes,
                                const void* v_dev, size_t v_bytes,
                                long* out_row) {
    if (!arena_ && !plan_only_) return false;
    const size_t total = k_bytes + v_bytes;
    if (arena_used_ + total > budget_bytes_) return false;
    if (arena_used_ + total > arena_cap_) return false;
    const long row = (long)arena_next_row_;
    if (!row_fits(row, total)) return false;
    if (!record_copy(row, k_dev, k_bytes, v_dev, v_bytes)) return false;
    *out_row = row;
    ++arena_next_row_;
    arena_used_ += total;
    return true;
}

long KVTileManager::arena_stage_rows(const char* k_first, size_t k_bytes, const char* v_first,
                                     size_t v_bytes, long n, long* out_slots) {
    const size_t total = k_bytes + v_bytes;
    const size_t stride = arena_row_stride_floats_ * sizeof(float);
    if (!plan_only_ || total == 0 || stride == 0 || n <= 0) {
        long m = 0;
        for (; m < n; ++m) {
            long row = -1;
            if (!arena_stage(k_first ? k_first + m * (long)k_bytes : nullptr, k_bytes,
                             v_first ? v_first + m * (long)v_bytes : nullptr, v_bytes, &row))
                break;
            if (out_slots) out_slots[m] = row;
        }
        return m;
    }
    // Plan-only: nothing to record, and each gate of arena_stage holds for
    // a prefix of the rows, so the staged count is the smallest prefix bound.
    auto fit = [&](size_t limit) -> size_t {
        return limit >= arena_used_ ? (limit - arena_used_) / total : 0;
    };
    size_t m = std::min(fit(budget_bytes_), fit(arena_cap_));
    const size_t last_row = arena_cap_ >= total ? (arena_cap_ - total) / stride : 0;
    const size_t by_row = (arena_cap_ >= total && last_row + 1 > arena_next_row_)
                              ? last_row + 1 - arena_next_row_ : 0;
    m = std::min(std::min(m, by_row), (size_t)n);
    if (out_slots)
        for (size_t i = 0; i < m; ++i) out_slots[i] = (long)(arena_next_row_ + i);
    arena_next_row_ += m;
    arena_used_ += m * total;
    return (long)m;
}

long KVTileManager::streaming_stage_rows(long row_first, const char* k_first, size_t k_bytes,
                                         const char* v_first, size_t v_bytes, long n,
                                         long* out_slots, long* copied) {
    long m = 0, c = 0;
    for (; m < n; ++m) {
        const long row = row_first + m;
        if (row == KvtmRowTable::kEmpty || row == KvtmRowTable::kTomb) break;
        // sticky hit (changed = false): the slot, no copy, no state change
        const long held = row_slot_.find(row);
        if (held >= 0) {
            if (out_slots) out_slots[m] = held;
            continue;
        }
        long slot = -1;
        bool restaged = false;
        if (!streaming_stage(row, k_first ? k_first + m * (long)k_bytes : nullptr,
                             k_bytes, v_first ? v_first + m * (long)v_bytes : nullptr, v_bytes,
                             false, &slot, &restaged))
            break;
        if (restaged) ++c;
        if (out_slots) out_slots[m] = slot;
    }
    if (copied) *copied = c;
    return m;
}

bool KVTileManager::arena_apply_window() {
    const bool ok = flush();
    if (!initialized_ || arena_used_ == 0 || arena_used_ > max_window_bytes_)
        return false;
    return ok;
}

void KVTileManager::arena_end_step() {
    flush();
    arena_next_row_ = 0;
    arena_used_ = 0;
}

void* KVTileManager::arena_device_ptr() const {
    flush();
    return arena_;
}

// ---- streaming mode (reference: src/kv_tile_manager.cu:141-219) ----

long KVTileManager::streaming_capacity_rows() const {
    const size_t stride = arena_row_stride_floats_ * sizeof(float);
    return stride ? (long)(arena_cap_ / stride) : 0;
}

bool KVTileManager::streaming_begin() {
    if (!arena_ && !plan_only_) return false;
    flush();
    row_slot_.clear();
    row_slot_.reserve((size_t)std::max<long>(0, streaming_capacity_rows()));
    free_slots_.clear();
    // Highest slot pushed first so the first pop hands out slot 0.
    for (long s = streaming_capacity_rows() - 1; s >= 0; --s) free_slots_.push_back(s);
    slot_high_water_ = -1;
    staged_bytes_ = 0;
    return true;
}

bool KVTileManager::streaming_stage(long row_id, const void* k_dev,
                                    size_t k_bytes, const void* v_dev,
                                    size_t v_bytes, bool changed,
                                    long* out_slot, bool* restaged) {
    if (row_id == KvtmRowTable::kEmpty || row_id == KvtmRowTable::kTomb) return false;
    const long held = row_slot_.find(row_id);
    if (held >= 0) {
        *out_slot = held;
        if (!changed) {
            *restaged = false;  // sticky hit: slot content still valid
            return true;
        }
        if (!row_fits(held, k_bytes + v_bytes)) return false;
        if (!record_copy(held, k_dev, k_bytes, v_dev, v_bytes)) return false;
        staged_bytes_ += k_bytes + v_bytes;
        *restaged = true;
        return true;
    }
    if (free_slots_.empty()) return false;  // capacity gate only
    const long slot = free_slots_.back();
    if (!row_fits(slot, k_bytes + v_bytes)) return false;
    if (!record_copy(slot, k_dev, k_bytes, v_dev, v_bytes)) return false;
    free_slots_.pop_back();
    row_slot_.insert(row_id, slot);
    staged_bytes_ += k_bytes + v_bytes;
    if (slot > slot_high_water_) slot_high_water_ = slot;
    *out_slot = slot;
    *restaged = true;
    return true;
}

bool KVTileManager::streaming_release(long row_id) {
    const long slot = row_slot_.erase(row_id);
    if (slot < 0) return false;
    free_slots_.push_back(slot);
    return true;
}

bool KVTileManager::streaming_apply_window() {
    const bool ok = flush();
    if (!initialized_ || slot_high_water_ < 0) return false;
    const size_t span = ((size_t)slot_high_water_ + 1) *
                        arena_row_stride_floats_ * sizeof(float);
    if (span > max_window_bytes_) return false;
    return ok;
}

void KVTileManager::streaming_end() {
    flush();
    row_slot_.clear();
    free_slots_.clear();
    slot_high_water_ = -1;
}
