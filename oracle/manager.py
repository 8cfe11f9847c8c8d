"""KVTileManager bookkeeping + driver plan model. TEST INFRASTRUCTURE ONLY.

ManagerModel restates the accounting and slot logic of the reference
manager (reference: src/kv_tile_manager.cu:49-219) with no device memory:
  window   admit -> -1 (uninitialised, id < 0, null ptr, 0 bytes, duplicate,
           bytes > max_window), 0 (used + bytes > budget) or 1   (:49-60)
  arena    rows handed out sequentially; refuse when used + k + v exceeds the
           budget or the capacity                                 (:104-121)
  stream   free list = [cap-1, ..., 0] popped from the back (slot 0 first),
           sticky hit = no copy unless changed, miss pops a slot, release
           pushes it back (LIFO reuse)                            (:141-200)

plan_frames() restates the driver's per-frame loop (reference:
src/run_policy_experiment.cu:156-274): selection, streaming release of
dropped tiles, map prefix reset to -1, staging in policy order with rows
ascending, map entries for staged rows. It returns, per frame, the selected
ids, the KVMap prefix, the list of (source row, arena row) copies, and the
number of fully staged tiles.

Pinned by (tests/test_oracle_pins.py): the reference's capacity/admission
scenario S1-S8 with its published numbers (reference:
tests/test_capacity_admission.py:80-148, configs/grounding_config.json:29-50)
and hand-derived slot sequences for the arena and streaming rules (LIFO
reuse, sticky hits, refusals leaving state unchanged, the intra-streaming
release quirk of src/run_policy_experiment.cu:180-185). The cross-frame
plan (tests/test_plan_pins.py): per-frame KVMap prefixes and copy lists
worked out by hand for recency and motion, arena and streaming, a sliding
window and a short last tile, each with planted mistakes (source row
without its frame term, release after staging, release in descending id
order) that must fail.
"""

from __future__ import annotations

import numpy as np

from . import policies

INVALID, REFUSED, ADMITTED = -1, 0, 1
RESIDENCY_LIMIT = 256 << 20


class ManagerModel:
    def __init__(self, budget: int, max_window: int):
        self.budget = budget
        self.max_window = max_window
        self.used = 0
        self.initialized = False
        self.active: dict[int, int] = {}
        self.arena_cap = 0
        self.stride_bytes = 0
        self.has_arena = False
        self.next_row = 0
        self.arena_used = 0
        self.row_slot: dict[int, int] = {}
        self.free_slots: list[int] = []
        self.high_water = -1
        self.staged_bytes = 0

    # window mode
    def init(self) -> bool:
        if self.budget > RESIDENCY_LIMIT:
            return False
        self.initialized = True
        return True

    def query_device_limit(self) -> int:
        return self.budget if self.initialized else 0

    def admit(self, tile_id: int, ptr: int, nbytes: int) -> int:
        if not self.initialized or tile_id < 0 or not ptr or nbytes == 0:
            return INVALID
        if tile_id in self.active:
            return INVALID
        if nbytes > self.max_window:
            return INVALID
        if self.used + nbytes > self.budget:
            return REFUSED
        self.active[tile_id] = nbytes
        self.used += nbytes
        return ADMITTED

    def release(self, tile_id: int) -> bool:
        if tile_id not in self.active:
            return False
        self.used -= self.active.pop(tile_id)
        return True

    def clear(self) -> None:
        self.active.clear()
        self.used = 0

    # arena mode
    def arena_init(self, cap_bytes: int, row_stride_floats: int) -> bool:
        if self.has_arena:
            return False
        self.has_arena = True
        self.arena_cap = cap_bytes
        self.stride_bytes = row_stride_floats * 4
        self.next_row = 0
        self.arena_used = 0
        return True

    def arena_begin_step(self) -> None:
        self.next_row = 0
        self.arena_used = 0

    def arena_stage(self, k_bytes: int, v_bytes: int):
        total = k_bytes + v_bytes
        if self.arena_used + total > self.budget:
            return None
        if self.arena_used + total > self.arena_cap:
            return None
        row = self.next_row
        self.next_row += 1
        self.arena_used += total
        return row

    # streaming mode
    def streaming_capacity(self) -> int:
        return self.arena_cap // self.stride_bytes if self.stride_bytes else 0

    def streaming_begin(self) -> bool:
        if not self.has_arena:
            return False
        self.row_slot.clear()
        self.free_slots = list(range(self.streaming_capacity() - 1, -1, -1))
        self.high_water = -1
        self.staged_bytes = 0
        return True

    def streaming_stage(self, row_id: int, k_bytes: int, v_bytes: int, changed: bool = False):
        """-> (ok, slot, restaged)"""
        if row_id in self.row_slot:
            slot = self.row_slot[row_id]
            if not changed:
                return True, slot, False
            self.staged_bytes += k_bytes + v_bytes
            return True, slot, True
        if not self.free_slots:
            return False, -1, False
        slot = self.free_slots.pop()
        self.row_slot[row_id] = slot
        self.staged_bytes += k_bytes + v_bytes
        self.high_water = max(self.high_water, slot)
        return True, slot, True

    def streaming_release(self, row_id: int) -> bool:
        if row_id not in self.row_slot:
            return False
        self.free_slots.append(self.row_slot.pop(row_id))
        return True

    def streaming_end(self) -> None:
        self.row_slot.clear()
        self.free_slots.clear()
        self.high_water = -1


PLANTS = ("drop_src_frame", "release_after_stage", "release_descending")


def plan_frames(policy: str, *, cross: bool, streaming: bool, frames: int, T: int, D: int,
                tile_tokens: int, set_aside: int, elem: int, scores_flat,
                window_frames: int = 0, _plant: str | None = None) -> list[dict]:
    """Per-frame driver plan; elem = bytes per element (4 fp32, 2 bf16).

    `_plant` plants one deliberate mistake for the pin tests (one of PLANTS):
    the source row without its frame term (tile rows of frame 0 instead of
    frame src_f), the streaming release after the frame's staging instead of
    before it, or the release walking dropped tiles in descending id order.
    """
    assert _plant is None or _plant in PLANTS
    num_tiles = (T + tile_tokens - 1) // tile_tokens
    persist = policy != "none"
    out = []
    if not persist:
        for f in range(frames):
            out.append(dict(ids=[], map=None, copies=[], staged_tiles=0))
        return out
    tile_bytes = tile_tokens * D * elem * 2
    slots = set_aside // tile_bytes
    mgr = ManagerModel(set_aside, set_aside)
    assert mgr.init()
    assert mgr.arena_init(set_aside, D * 2 * elem // 4)
    if streaming:
        mgr.streaming_begin()
    scores_flat = np.asarray(scores_flat, dtype=np.float32).reshape(-1)
    row_bytes = D * elem
    h_map = np.full(frames * T, -1, dtype=np.int64)
    prev_selected = None
    for f in range(frames):
        kb_frame = 0
        if cross and window_frames and f + 1 > window_frames:
            kb_frame = f + 1 - window_frames
        if cross:
            first = kb_frame * num_tiles
            n = (f + 1) * num_tiles - first
            ids = policies.select_range(policy, scores_flat, first, n, slots,
                                        tiles_per_frame=num_tiles, total_frames=frames)
        else:
            ids = policies.select(policy, scores_flat[f * num_tiles:(f + 1) * num_tiles],
                                  num_tiles, slots, tiles_per_frame=num_tiles,
                                  total_frames=frames)
        selected = np.zeros((f + 1) * num_tiles, dtype=bool)
        for i in ids:
            if 0 <= i < selected.size:
                selected[i] = True
        def release_dropped():
            order = range(prev_selected.size)
            if _plant == "release_descending":
                order = reversed(order)
            for gid in order:
                if not prev_selected[gid]:
                    continue
                if gid < selected.size and selected[gid]:
                    continue
                src_f = gid // num_tiles if cross else f
                tile = gid % num_tiles if cross else gid
                t0 = tile * tile_tokens
                c = min(tile_tokens, T - t0)
                for r in range(c):
                    mgr.streaming_release(src_f * T + t0 + r)

        if streaming and f > 0 and _plant != "release_after_stage":
            release_dropped()
        mgr.arena_begin_step()
        h_map[:(f + 1) * T] = -1
        copies = []
        staged_tiles = 0
        for gid in ids:
            src_f = gid // num_tiles if cross else f
            tile = gid % num_tiles if cross else gid
            if src_f >= frames:
                continue  # uniform id past the last frame: rows outside K/V
            t0 = tile * tile_tokens
            c = min(tile_tokens, T - t0)
            ok = True
            r = 0
            while r < c and ok:
                row_id = (0 if _plant == "drop_src_frame" else src_f * T) + t0 + r
                if streaming:
                    ok, slot, restaged = mgr.streaming_stage(row_id, row_bytes, row_bytes)
                    if ok:
                        h_map[row_id] = slot
                        if restaged:
                            copies.append((row_id, slot))
                else:
                    slot = mgr.arena_stage(row_bytes, row_bytes)
                    ok = slot is not None
                    if ok:
                        h_map[row_id] = slot
                        copies.append((row_id, slot))
                r += 1
            if ok:
                staged_tiles += 1
        if streaming and f > 0 and _plant == "release_after_stage":
            release_dropped()
        if streaming:
            prev_selected = selected
        else:
            mgr.arena_begin_step()
        out.append(dict(ids=list(ids), map=h_map[:(f + 1) * T].copy(), copies=copies,
                        staged_tiles=staged_tiles,
                        staged_bytes=mgr.staged_bytes if streaming else None))
    return out
