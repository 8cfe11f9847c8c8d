"""Python mirror of the C++ interface of the hot path, over the C-ABI.

Names, argument meaning and return conventions follow the reference
classes/functions so host code and tests read like the reference's own:

* ``KVTileManager``  (reference: src/kv_tile_manager.h:21-66)
* ``TileGatingPolicy`` and ``make_policy`` (reference: src/tile_gating_policy.h)
* ``TileLayout``     (reference: src/tile_layout.h:13-31)
* ``attn_forward_launcher`` / ``attn_forward_single_frame``
  (reference: src/attn_kernel.h:15-29) plus bf16 / window / range forms
* ``FramePipeline``  (the driver loop of src/run_policy_experiment.cu:136-283)

Device buffers are passed as torch tensors (their ``data_ptr()``) or raw
integer addresses; torch is only plumbing for memory and streams.
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np

from . import _lib

KVTM_ADMITTED, KVTM_REFUSED_BUDGET, KVTM_INVALID = 1, 0, -1
FP32, BF16 = 0, 1
HEAD_DIM = 128
COLD_ROWS_NT = 1  # kvp_attn_forward_frames flag (KVP_ATTN_COLD_ROWS_NT)


def _ptr(x) -> int | None:
    """Device address of a torch tensor / int / None."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return int(x.data_ptr())


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed: {_lib.last_error()}")


class TileLayout:
    """Host-side tile arithmetic, evaluated by the library's C helpers."""

    def __init__(self, tokens_per_frame: int, tile_tokens: int):
        self.tokens_per_frame = tokens_per_frame
        self.tile_tokens = tile_tokens
        self.tiles_per_frame = int(
            _lib.load().kvtm_layout_tiles_per_frame(tokens_per_frame, tile_tokens))

    def tile_start(self, tile_id: int) -> int:
        return int(_lib.load().kvtm_layout_tile_start(self.tokens_per_frame, self.tile_tokens,
                                                      tile_id))

    def tile_count(self, tile_id: int) -> int:
        return int(_lib.load().kvtm_layout_tile_count(self.tokens_per_frame, self.tile_tokens,
                                                      tile_id))

    def tile_of_token(self, token: int) -> int:
        return token // self.tile_tokens


class TileGatingPolicy:
    """One of none / uniform / recency / motion / reuse_weighted."""

    def __init__(self, name: str, tiles_per_frame: int = 1, total_frames: int = 1):
        self._lib = _lib.load()
        self._h = self._lib.kvp_policy_create(name.encode(), tiles_per_frame, total_frames)
        if not self._h:
            raise ValueError(f"unknown policy {name!r}")

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.kvp_policy_destroy(h)
            self._h = None

    def name(self) -> str:
        return self._lib.kvp_policy_name(self._h).decode()

    def select(self, scores: Sequence[float] | np.ndarray | None, num_candidates: int,
               max_tiles: int) -> list[int]:
        sc = _as_f32(scores, num_candidates)
        out = (ctypes.c_long * max(1, max_tiles))()
        n = self._lib.kvp_policy_select(self._h, sc, num_candidates, max_tiles, out)
        return [int(out[i]) for i in range(n)]

    def select_range(self, scores_flat, first_id: int, num_candidates: int,
                     max_tiles: int) -> list[int]:
        sc = _as_f32(scores_flat, first_id + num_candidates)
        out = (ctypes.c_long * max(1, max_tiles))()
        n = self._lib.kvp_policy_select_range(self._h, sc, first_id, num_candidates,
                                              max_tiles, out)
        return [int(out[i]) for i in range(n)]


def make_policy(name: str, tiles_per_frame: int = 1, total_frames: int = 1) -> TileGatingPolicy:
    return TileGatingPolicy(name, tiles_per_frame, total_frames)


def _as_f32(scores, n: int):
    if scores is None:
        return ctypes.cast(None, _lib.c_float_p)
    arr = np.ascontiguousarray(np.asarray(scores, dtype=np.float32))
    if arr.size < n:
        raise ValueError(f"need {n} scores, got {arr.size}")
    buf = (ctypes.c_float * max(1, arr.size)).from_buffer_copy(arr.tobytes() or b"\0\0\0\0")
    return buf


class KVTileManager:
    """Budget accounting + hot arena (see include/kv_tile_manager.h)."""

    def __init__(self, budget_bytes: int, max_window_bytes: int):
        self._lib = _lib.load()
        self._h = self._lib.kvtm_create(budget_bytes, max_window_bytes)
        if not self._h:
            raise RuntimeError("kvtm_create failed")

    def close(self):
        if getattr(self, "_h", None):
            self._lib.kvtm_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def handle(self) -> int:
        return self._h

    # window mode
    def init(self) -> bool:
        return self._lib.kvtm_init(self._h) == 1

    def query_device_limit(self) -> int:
        return int(self._lib.kvtm_query_limit(self._h))

    def admit(self, tile_id: int, ptr: int, nbytes: int) -> int:
        return int(self._lib.kvtm_admit(self._h, tile_id, ptr, nbytes))

    def release(self, tile_id: int) -> bool:
        return self._lib.kvtm_release(self._h, tile_id) == 1

    def clear(self) -> None:
        self._lib.kvtm_clear(self._h)

    def persisted_bytes(self) -> int:
        return int(self._lib.kvtm_persisted_bytes(self._h))

    def persisted_tiles(self) -> int:
        return int(self._lib.kvtm_persisted_tiles(self._h))

    def is_persisted(self, tile_id: int) -> bool:
        return self._lib.kvtm_is_persisted(self._h, tile_id) == 1

    # arena mode
    def arena_init(self, capacity_bytes: int, row_stride_floats: int) -> bool:
        return self._lib.kvtm_arena_init(self._h, capacity_bytes, row_stride_floats) == 1

    def arena_attach(self, dev_ptr, capacity_bytes: int, row_stride_floats: int) -> bool:
        return self._lib.kvtm_arena_attach(self._h, _ptr(dev_ptr), capacity_bytes,
                                           row_stride_floats) == 1

    def arena_begin_step(self) -> None:
        self._lib.kvtm_arena_begin(self._h)

    def arena_stage(self, k_dev: int, k_bytes: int, v_dev: int, v_bytes: int) -> int | None:
        row = ctypes.c_long(-1)
        ok = self._lib.kvtm_arena_stage(self._h, k_dev, k_bytes, v_dev, v_bytes,
                                        ctypes.byref(row))
        return int(row.value) if ok == 1 else None

    def arena_apply_window(self) -> bool:
        return self._lib.kvtm_arena_window(self._h) == 1

    def arena_end_step(self) -> None:
        self._lib.kvtm_arena_end(self._h)

    def arena_used_bytes(self) -> int:
        return int(self._lib.kvtm_arena_used(self._h))

    def arena_device_ptr(self) -> int:
        return int(self._lib.kvtm_arena_ptr(self._h) or 0)

    # streaming mode
    def streaming_begin(self) -> bool:
        return self._lib.kvtm_streaming_begin(self._h) == 1

    def streaming_stage(self, row_id: int, k_dev: int, k_bytes: int, v_dev: int, v_bytes: int,
                        changed: bool = False):
        slot = ctypes.c_long(-1)
        restaged = ctypes.c_int(0)
        ok = self._lib.kvtm_streaming_stage(self._h, row_id, k_dev, k_bytes, v_dev, v_bytes,
                                            1 if changed else 0, ctypes.byref(slot),
                                            ctypes.byref(restaged))
        return (ok == 1, int(slot.value), bool(restaged.value))

    def streaming_release(self, row_id: int) -> bool:
        return self._lib.kvtm_streaming_release(self._h, row_id) == 1

    def streaming_apply_window(self) -> bool:
        return self._lib.kvtm_streaming_window(self._h) == 1

    def streaming_end(self) -> None:
        self._lib.kvtm_streaming_end(self._h)

    def streaming_staged_bytes(self) -> int:
        return int(self._lib.kvtm_streaming_staged_bytes(self._h))

    def streaming_high_water(self) -> int:
        return int(self._lib.kvtm_streaming_high_water(self._h))

    def streaming_capacity(self) -> int:
        return int(self._lib.kvtm_streaming_capacity(self._h))

    def flush(self) -> bool:
        return self._lib.kvtm_flush(self._h) == 1

    def pending_copies(self) -> int:
        return int(self._lib.kvtm_pending_copies(self._h))

    def set_stream(self, stream: int | None) -> None:
        self._lib.kvtm_set_stream(self._h, stream)


# ---------------------------------------------------------------- attention

def attn_forward_launcher(q, k, v, arena, kvmap, out, frames: int, T: int, D: int, heads: int,
                          remap: bool) -> None:
    """fp32, reference semantics (src/gated_attention_kernel.cu:141-168)."""
    lib = _lib.load()
    _check(lib.kvp_attn_forward_launcher(_ptr(q), _ptr(k), _ptr(v), _ptr(arena), _ptr(kvmap),
                                         _ptr(out), frames, T, D, heads, 1 if remap else 0),
           "attn_forward_launcher")


def attn_forward_single_frame(q_f, k, v, arena, kvmap_f, out_f, T: int, D: int, heads: int,
                              cross: int, frame_idx: int, window_frames: int = 0) -> None:
    """fp32 one-frame launch (src/gated_attention_kernel.cu:170-184)."""
    lib = _lib.load()
    if window_frames:
        rc = lib.kvp_attn_forward_single_frame_window(
            _ptr(q_f), _ptr(k), _ptr(v), _ptr(arena), _ptr(kvmap_f), _ptr(out_f), T, D, heads,
            cross, frame_idx, window_frames)
    else:
        rc = lib.kvp_attn_forward_single_frame(_ptr(q_f), _ptr(k), _ptr(v), _ptr(arena),
                                               _ptr(kvmap_f), _ptr(out_f), T, D, heads, cross,
                                               frame_idx)
    _check(rc, "attn_forward_single_frame")


def attn_forward_launcher_bf16(q, k, v, arena, kvmap, out, frames: int, T: int, D: int,
                               heads: int, remap: bool) -> None:
    lib = _lib.load()
    _check(lib.kvp_attn_forward_launcher_bf16(_ptr(q), _ptr(k), _ptr(v), _ptr(arena),
                                              _ptr(kvmap), _ptr(out), frames, T, D, heads,
                                              1 if remap else 0),
           "attn_forward_launcher_bf16")


def attn_forward_single_frame_bf16(q_f, k, v, arena, kvmap_f, out_f, T: int, D: int, heads: int,
                                   cross: int, frame_idx: int, window_frames: int = 0) -> None:
    lib = _lib.load()
    _check(lib.kvp_attn_forward_single_frame_bf16(_ptr(q_f), _ptr(k), _ptr(v), _ptr(arena),
                                                  _ptr(kvmap_f), _ptr(out_f), T, D, heads,
                                                  cross, frame_idx, window_frames),
           "attn_forward_single_frame_bf16")


def attn_forward_range(dtype: int, q, k, v, arena, kvmap, out, nq: int, D: int, heads: int,
                       key_begin: int, key_end: int, stream: int | None = None) -> None:
    lib = _lib.load()
    _check(lib.kvp_attn_forward_range(dtype, _ptr(q), _ptr(k), _ptr(v), _ptr(arena),
                                      _ptr(kvmap), _ptr(out), nq, D, heads, key_begin, key_end,
                                      stream),
           "attn_forward_range")


def attn_forward_frames(dtype: int, q, k, v, arena, kvmap, out, frames: int, T: int, D: int,
                        heads: int, *, cross: bool, window_frames: int = 0,
                        arena_frame_bytes: int = 0, map_frame_stride: int = 0,
                        cold_rows_nt: bool = False, stream: int | None = None) -> None:
    """All frames of a layer in one launch (frame f reads arena region f and
    KVMap slice f); see kvp_attn_forward_frames in kvp_c_api.h."""
    flags = COLD_ROWS_NT if cold_rows_nt else 0
    _check(_lib.load().kvp_attn_forward_frames(dtype, _ptr(q), _ptr(k), _ptr(v), _ptr(arena),
                                               arena_frame_bytes, _ptr(kvmap), map_frame_stride,
                                               _ptr(out), frames, T, D, heads, int(cross),
                                               window_frames, flags, stream),
           "attn_forward_frames")


def attn_forward_frames_gd(q, k, v, arena, kvmap, gdesc, out, frames: int, T: int, D: int,
                           heads: int, *, cross: bool, gd_frame_stride: int,
                           window_frames: int = 0, arena_frame_bytes: int = 0,
                           map_frame_stride: int = 0, stream: int | None = None) -> None:
    """attn_forward_frames for bf16 with the map's group descriptors (frame
    f's table at gdesc + 8 * f * gd_frame_stride bytes); see
    kvp_attn_forward_frames_gd in kvp_c_api.h."""
    _check(_lib.load().kvp_attn_forward_frames_gd(_ptr(q), _ptr(k), _ptr(v), _ptr(arena),
                                                  arena_frame_bytes, _ptr(kvmap),
                                                  map_frame_stride, _ptr(gdesc), gd_frame_stride,
                                                  _ptr(out), frames, T, D, heads, int(cross),
                                                  window_frames, stream),
           "attn_forward_frames_gd")


def attn_group_desc(kvmap, key_begin: int, key_end: int, D: int) -> np.ndarray:
    """Group-descriptor table of one frame's KVMap slice (host int64 array
    indexed by key row) over the key range [key_begin, key_end): uint32
    array [entries, 2]; see kvp_attn_group_desc in kvp_c_api.h."""
    m = np.ascontiguousarray(kvmap, dtype=np.int64)
    if key_end > len(m):
        raise ValueError("attn_group_desc: key range past the map")
    lib = _lib.load()
    mp = m.ctypes.data_as(_lib.c_long_p)
    n = int(lib.kvp_attn_group_desc(mp, key_begin, key_end, D, None, 0))
    if n < 0:
        raise RuntimeError(f"attn_group_desc: {_lib.last_error()}")
    out = np.zeros((n, 2), dtype=np.uint32)
    if n:
        _check(0 if lib.kvp_attn_group_desc(mp, key_begin, key_end, D, out.ctypes.data, n) == n
               else 1, "attn_group_desc")
    return out


def attn_splits(dtype: int, nq: int, heads: int, frames: int, span: int) -> int:
    return int(_lib.load().kvp_attn_splits(dtype, nq, heads, frames, span))


def set_stream(stream: int | None) -> None:
    _lib.load().kvp_set_stream(stream)


def device_sync() -> None:
    _check(_lib.load().kvp_device_sync(), "device sync")


# ---------------------------------------------------------------- pipeline

class FramePipeline:
    """Per-frame select -> release -> stage -> map -> attention loop."""

    def __init__(self, policy: str, *, cross: bool, streaming: bool, frames: int, T: int,
                 D: int, heads: int, tile_tokens: int = 16, set_aside_bytes: int = 0,
                 dtype: int = FP32, window_frames: int = 0, plan_only: bool = False):
        self._lib = _lib.load()
        self.frames, self.T, self.D, self.heads = frames, T, D, heads
        self.tile_tokens = tile_tokens
        self.cross = cross
        self.num_tiles = (T + tile_tokens - 1) // tile_tokens
        self._h = self._lib.kvp_pipeline_create(policy.encode(), int(cross), int(streaming),
                                                frames, T, D, heads, tile_tokens,
                                                set_aside_bytes, dtype, window_frames,
                                                int(plan_only))
        if not self._h:
            raise RuntimeError(f"kvp_pipeline_create failed: {_lib.last_error()}")
        self._scores = None

    def close(self):
        if getattr(self, "_h", None):
            self._lib.kvp_pipeline_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    def set_scores(self, scores_flat) -> None:
        if scores_flat is None:
            self._scores = None
            return
        arr = np.ascontiguousarray(np.asarray(scores_flat, dtype=np.float32).reshape(-1))
        self._scores_np = arr
        self._scores = arr.ctypes.data_as(_lib.c_float_p)

    def set_stream(self, stream: int | None) -> None:
        self._lib.kvp_pipeline_set_stream(self._h, stream)

    def set_cold_rows_nt(self, on: bool) -> None:
        """Attention launches load original (non-arena) K/V rows non-temporally."""
        self._lib.kvp_pipeline_set_cold_rows_nt(self._h, int(bool(on)))

    def step(self, f: int, q=None, k=None, v=None, out=None) -> None:
        _check(self._lib.kvp_pipeline_step(self._h, f, _ptr(q), _ptr(k), _ptr(v), _ptr(out),
                                           self._scores), f"pipeline step {f}")

    def run(self, q=None, k=None, v=None, out=None) -> None:
        """A whole layer: one staging launch that copies every row any frame
        maps into the layer arena (once) and writes each frame's KVMap slice,
        then one attention launch over all frames. Plan-only pipelines apply
        the staging on the host (layer_plan_map / layer_plan_sources)."""
        _check(self._lib.kvp_pipeline_run(self._h, _ptr(q), _ptr(k), _ptr(v), _ptr(out),
                                          self._scores), "pipeline run")

    def selected(self) -> list[int]:
        cap = self.frames * self.num_tiles + 64
        buf = (ctypes.c_long * cap)()
        n = self._lib.kvp_pipeline_selected(self._h, buf, cap)
        return [int(buf[i]) for i in range(min(n, cap))]

    def host_map(self) -> np.ndarray:
        n = self.frames * self.T
        buf = np.empty(n, dtype=np.int64)
        got = self._lib.kvp_pipeline_map(self._h, buf.ctypes.data_as(_lib.c_long_p), n)
        return buf[:got] if got < n else buf

    def slots(self) -> int:
        return int(self._lib.kvp_pipeline_slots(self._h))

    def staged_tiles(self) -> int:
        return int(self._lib.kvp_pipeline_staged_tiles(self._h))

    def staged_bytes(self) -> int:
        return int(self._lib.kvp_pipeline_staged_bytes(self._h))

    def copy_rows(self) -> int:
        return int(self._lib.kvp_pipeline_copy_rows(self._h))

    def arena_ptr(self) -> int:
        return int(self._lib.kvp_pipeline_arena(self._h) or 0)

    def device_map_ptr(self) -> int:
        return int(self._lib.kvp_pipeline_device_map(self._h) or 0)

    # layer mode (after run): the arena all frames share, frame f's KVMap
    # slice, and the rows the last run copied
    def layer_arena_ptr(self) -> int:
        return int(self._lib.kvp_pipeline_layer_arena(self._h) or 0)

    def layer_copied_rows(self) -> int:
        return int(self._lib.kvp_pipeline_layer_copied_rows(self._h))

    # plan-only pipelines, after run(): the layer map slice of frame f and
    # the K/V row of each physical row, as the staging launch would leave them
    def layer_plan_map(self, f: int) -> np.ndarray:
        n = int(self._lib.kvp_pipeline_layer_plan_map(self._h, f, None, 0))
        if n < 0:
            raise RuntimeError("layer_plan_map: not a plan-only pipeline after run()")
        buf = np.empty(n, dtype=np.int64)
        self._lib.kvp_pipeline_layer_plan_map(self._h, f, buf.ctypes.data_as(_lib.c_long_p), n)
        return buf

    def layer_plan_sources(self) -> np.ndarray:
        n = int(self._lib.kvp_pipeline_layer_plan_sources(self._h, None, 0))
        if n < 0:
            raise RuntimeError("layer_plan_sources: not a plan-only pipeline after run()")
        buf = np.empty(n, dtype=np.int64)
        self._lib.kvp_pipeline_layer_plan_sources(self._h, buf.ctypes.data_as(_lib.c_long_p), n)
        return buf

    def layer_map_ptr(self, f: int = 0) -> int:
        base = int(self._lib.kvp_pipeline_layer_map(self._h) or 0)
        return base + 8 * f * int(self._lib.kvp_pipeline_layer_map_stride(self._h)) if base else 0

    def layer_map_stride(self) -> int:
        return int(self._lib.kvp_pipeline_layer_map_stride(self._h))

    def layer_arena_bytes(self) -> int:
        return int(self._lib.kvp_pipeline_layer_arena_bytes(self._h))

    # group descriptors of the layer map (bf16 layer runs)
    def layer_gd_ptr(self) -> int:
        return int(self._lib.kvp_pipeline_layer_gd(self._h) or 0)

    def layer_gd_stride(self) -> int:
        return int(self._lib.kvp_pipeline_layer_gd_stride(self._h))

    def layer_plan_gd(self, f: int) -> np.ndarray:
        """Plan-only, after run(): frame f's descriptor table, uint32 [stride, 2]."""
        n = int(self._lib.kvp_pipeline_layer_plan_gd(self._h, f, None, 0))
        if n < 0:
            raise RuntimeError("layer_plan_gd: not a plan-only pipeline after run()")
        buf = np.zeros((n, 2), dtype=np.uint32)
        if n:
            self._lib.kvp_pipeline_layer_plan_gd(self._h, f, buf.ctypes.data, n)
        return buf

    def layer_attention(self, q, k, v, out) -> None:
        """The last run()'s attention launch again, alone (same arena, map
        slices and descriptors) on the pipeline's stream."""
        _check(self._lib.kvp_pipeline_layer_attention(self._h, _ptr(q), _ptr(k), _ptr(v),
                                                      _ptr(out)), "pipeline layer_attention")
