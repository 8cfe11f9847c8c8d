"""ctypes binding of libkvpersist.so (the C-ABI declared in include/*.h).

The library is built in-tree by ``make -C cuda-kv-persistence_amd`` (or
``__graft_entry__.build()``). Loading fails loudly when it is missing: there
is no CPU fallback for any device entry point.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parents[1]
LIB_PATH = PKG_ROOT / "lib" / "libkvpersist.so"
CLI_PATH = PKG_ROOT / "bin" / "policy_experiment"

c_long = ctypes.c_long
c_int = ctypes.c_int
c_void_p = ctypes.c_void_p
c_char_p = ctypes.c_char_p
c_float_p = ctypes.POINTER(ctypes.c_float)
c_long_p = ctypes.POINTER(ctypes.c_long)
c_int_p = ctypes.POINTER(ctypes.c_int)
c_size_t = ctypes.c_size_t
c_double = ctypes.c_double

# name -> (restype, argtypes); every symbol declared in include/*.h.
SIGNATURES = {
    # KVTileManager facade (reference: src/kv_tile_manager.cu:223-341)
    "kvtm_create": (c_void_p, [c_long, c_long]),
    "kvtm_destroy": (None, [c_void_p]),
    "kvtm_init": (c_int, [c_void_p]),
    "kvtm_query_limit": (c_long, [c_void_p]),
    "kvtm_admit": (c_int, [c_void_p, c_long, c_void_p, c_long]),
    "kvtm_release": (c_int, [c_void_p, c_long]),
    "kvtm_clear": (None, [c_void_p]),
    "kvtm_persisted_bytes": (c_long, [c_void_p]),
    "kvtm_persisted_tiles": (c_int, [c_void_p]),
    "kvtm_dev_alloc": (c_void_p, [c_long]),
    "kvtm_dev_free": (None, [c_void_p]),
    "kvtm_arena_init": (c_int, [c_void_p, c_long, c_long]),
    "kvtm_arena_begin": (None, [c_void_p]),
    "kvtm_arena_stage": (c_int, [c_void_p, c_void_p, c_long, c_void_p, c_long, c_long_p]),
    "kvtm_arena_window": (c_int, [c_void_p]),
    "kvtm_arena_end": (None, [c_void_p]),
    "kvtm_arena_used": (c_long, [c_void_p]),
    "kvtm_arena_ptr": (c_void_p, [c_void_p]),
    "kvtm_streaming_begin": (c_int, [c_void_p]),
    "kvtm_streaming_stage": (c_int, [c_void_p, c_long, c_void_p, c_long, c_void_p, c_long,
                                     c_int, c_long_p, c_int_p]),
    "kvtm_streaming_release": (c_int, [c_void_p, c_long]),
    "kvtm_streaming_window": (c_int, [c_void_p]),
    "kvtm_streaming_end": (None, [c_void_p]),
    "kvtm_streaming_staged_bytes": (c_long, [c_void_p]),
    "kvtm_layout_tiles_per_frame": (c_long, [c_int, c_int]),
    "kvtm_layout_tile_start": (c_long, [c_int, c_int, c_long]),
    "kvtm_layout_tile_count": (c_int, [c_int, c_int, c_long]),
    "kvtm_arena_attach": (c_int, [c_void_p, c_void_p, c_long, c_long]),
    "kvtm_flush": (c_int, [c_void_p]),
    "kvtm_set_stream": (None, [c_void_p, c_void_p]),
    "kvtm_is_persisted": (c_int, [c_void_p, c_long]),
    "kvtm_streaming_high_water": (c_long, [c_void_p]),
    "kvtm_streaming_capacity": (c_long, [c_void_p]),
    "kvtm_pending_copies": (c_long, [c_void_p]),
    # policies (reference: src/tile_gating_policy.h:8-68)
    "kvp_policy_create": (c_void_p, [c_char_p, c_int, c_int]),
    "kvp_policy_destroy": (None, [c_void_p]),
    "kvp_policy_name": (c_char_p, [c_void_p]),
    "kvp_policy_select": (c_int, [c_void_p, c_float_p, c_int, c_int, c_long_p]),
    "kvp_policy_select_range": (c_int, [c_void_p, c_float_p, c_long, c_int, c_int, c_long_p]),
    # attention (reference: src/attn_kernel.h:15-29)
    "kvp_attn_forward_launcher": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                          c_void_p, c_int, c_int, c_int, c_int, c_int]),
    "kvp_attn_forward_single_frame": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                              c_void_p, c_int, c_int, c_int, c_int, c_int]),
    "kvp_attn_forward_launcher_bf16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                               c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                               c_int]),
    "kvp_attn_forward_single_frame_bf16": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                   c_void_p, c_void_p, c_int, c_int, c_int,
                                                   c_int, c_int, c_int]),
    "kvp_attn_forward_single_frame_window": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                                     c_void_p, c_void_p, c_int, c_int, c_int,
                                                     c_int, c_int, c_int]),
    "kvp_attn_forward_range": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p, c_int, c_int, c_int, c_long, c_long, c_void_p]),
    "kvp_attn_forward_range_noalloc": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                               c_void_p, c_void_p, c_int, c_int, c_int, c_long,
                                               c_long, c_void_p]),
    "kvp_attn_forward_frames": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_long,
                                        c_void_p, c_long, c_void_p, c_int, c_int, c_int, c_int,
                                        c_int, c_int, c_int, c_void_p]),
    "kvp_attn_forward_frames_gd": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_long,
                                           c_void_p, c_long, c_void_p, c_long, c_void_p, c_int,
                                           c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "kvp_attn_group_desc": (c_long, [c_long_p, c_long, c_long, c_int, c_void_p, c_long]),
    "kvp_attn_workspace_release": (c_int, [c_void_p]),
    "kvp_attn_workspace_count": (c_long, []),
    "kvp_set_stream": (None, [c_void_p]),
    "kvp_get_stream": (c_void_p, []),
    "kvp_last_error": (c_char_p, []),
    "kvp_device_count": (c_int, []),
    "kvp_attn_block_queries": (c_int, [c_int]),
    "kvp_attn_block_keys": (c_int, [c_int]),
    "kvp_attn_splits": (c_int, [c_int, c_int, c_int, c_int, c_long]),
    # device layer
    "kvp_dev_alloc": (c_void_p, [c_size_t]),
    "kvp_dev_free": (None, [c_void_p]),
    "kvp_memcpy_h2d": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "kvp_memcpy_d2h": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "kvp_memcpy_d2d": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "kvp_stream_sync": (c_int, [c_void_p]),
    "kvp_device_sync": (c_int, []),
    "kvp_stager_create": (c_void_p, []),
    "kvp_stager_destroy": (None, [c_void_p]),
    "kvp_stage_run": (c_int, [c_void_p, c_void_p, c_long, c_void_p, c_long, c_void_p, c_long,
                              c_void_p, c_void_p, c_long, c_void_p]),
    # frame pipeline (reference: src/run_policy_experiment.cu:136-283)
    "kvp_pipeline_create": (c_void_p, [c_char_p, c_int, c_int, c_int, c_int, c_int, c_int,
                                       c_int, c_long, c_int, c_int, c_int]),
    "kvp_pipeline_destroy": (None, [c_void_p]),
    "kvp_pipeline_set_stream": (c_int, [c_void_p, c_void_p]),
    "kvp_pipeline_set_cold_rows_nt": (c_int, [c_void_p, c_int]),
    "kvp_pipeline_step": (c_int, [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_float_p]),
    "kvp_pipeline_run": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_float_p]),
    "kvp_pipeline_selected": (c_int, [c_void_p, c_long_p, c_int]),
    "kvp_pipeline_map": (c_long, [c_void_p, c_long_p, c_long]),
    "kvp_pipeline_slots": (c_long, [c_void_p]),
    "kvp_pipeline_staged_tiles": (c_long, [c_void_p]),
    "kvp_pipeline_staged_bytes": (c_long, [c_void_p]),
    "kvp_pipeline_copy_rows": (c_long, [c_void_p]),
    "kvp_pipeline_arena": (c_void_p, [c_void_p]),
    "kvp_pipeline_device_map": (c_void_p, [c_void_p]),
    "kvp_pipeline_manager": (c_void_p, [c_void_p]),
    "kvp_pipeline_layer_arena": (c_void_p, [c_void_p]),
    "kvp_pipeline_layer_map": (c_void_p, [c_void_p]),
    "kvp_pipeline_layer_map_stride": (c_long, [c_void_p]),
    "kvp_pipeline_layer_copied_rows": (c_long, [c_void_p]),
    "kvp_pipeline_layer_plan_map": (c_long, [c_void_p, c_int, c_long_p, c_long]),
    "kvp_pipeline_layer_plan_sources": (c_long, [c_void_p, c_long_p, c_long]),
    "kvp_pipeline_layer_plan_gd": (c_long, [c_void_p, c_int, c_void_p, c_long]),
    "kvp_pipeline_layer_arena_bytes": (c_long, [c_void_p]),
    "kvp_pipeline_layer_gd": (c_void_p, [c_void_p]),
    "kvp_pipeline_layer_gd_stride": (c_long, [c_void_p]),
    "kvp_pipeline_layer_attention": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p,
                                             c_void_p]),
    # upstream K/V producer (reference: src/backbone.py:8-67), include/kvp_producer.h
    "kvp_layer_norm": (c_int, [c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_long,
                               c_int, ctypes.c_float, c_void_p]),
    "kvp_linear": (c_int, [c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_long, c_int,
                           c_int, c_int, c_void_p]),
    "kvp_proj_gemm": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                              c_int, c_long, c_int, c_int, c_int, c_int, c_int, c_void_p]),
    "kvp_qkv_project": (c_int, [c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                c_void_p, c_void_p, c_void_p, c_void_p, c_long, c_int,
                                c_void_p]),
    "kvp_backbone_create": (c_void_p, [c_int, c_int, c_int, c_int, c_int, c_int,
                                       ctypes.c_ulong]),
    "kvp_backbone_destroy": (None, [c_void_p]),
    "kvp_backbone_param_count": (c_long, [c_void_p]),
    "kvp_backbone_num_tensors": (c_int, [c_void_p]),
    "kvp_backbone_tensor_name": (c_char_p, [c_void_p, c_int]),
    "kvp_backbone_param_info": (c_int, [c_void_p, c_char_p, ctypes.POINTER(c_void_p), c_long_p,
                                        c_int_p]),
    "kvp_backbone_set_param": (c_int, [c_void_p, c_char_p, c_float_p, c_long]),
    "kvp_backbone_get_param": (c_int, [c_void_p, c_char_p, c_float_p, c_long]),
    "kvp_backbone_forward": (c_int, [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p,
                                     c_void_p, c_long, c_void_p]),
    # upstream motion producer (reference: traces/gen_motion_from_video.py:61-67,104-126)
    "kvp_farneback_workspace_bytes": (c_long, [c_int, c_int, c_int, c_double, c_int]),
    "kvp_farneback_flows": (c_int, [c_void_p, c_int, c_int, c_int, c_double, c_int, c_int, c_int,
                                    c_int, c_double, c_int, c_void_p, c_long, c_void_p,
                                    c_void_p]),
    "kvp_farneback_flow": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_double, c_int,
                                   c_int, c_int, c_int, c_double, c_int, c_void_p, c_long,
                                   c_void_p]),
    "kvp_farneback_profile": (c_int, [c_void_p, c_int, c_int, c_int, c_double, c_int, c_int,
                                      c_int, c_int, c_double, c_int, c_void_p, c_long, c_void_p,
                                      c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p]),
    "kvp_motion_change_rates": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int,
                                        c_void_p, c_void_p, c_void_p]),
}

_LIB = None


class LibraryMissing(RuntimeError):
    pass


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load libkvpersist.so and attach every signature; raise if absent."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise LibraryMissing(
            f"{p} is not built; run `make -C {PKG_ROOT}` or __graft_entry__.build()")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if a declared symbol is missing
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def last_error() -> str:
    return load().kvp_last_error().decode(errors="replace")
