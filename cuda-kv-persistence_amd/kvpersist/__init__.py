"""kvpersist: MI355X-native KVMap-indirected attention + KV arena.

Python side of ``cuda-kv-persistence_amd``: a ctypes mirror of the C++ API
(include/*.h), the upstream K/V producer (``kvpersist.backbone``) and the
synthetic workload generators used by the benchmark.
All compute runs in libkvpersist.so (gfx950 HIP); importing this package
never falls back to a CPU implementation.
"""

from . import backbone
from ._lib import CLI_PATH, LIB_PATH, PKG_ROOT, LibraryMissing, last_error, load
from .api import (BF16, FP32, HEAD_DIM, KVTM_ADMITTED, KVTM_INVALID, KVTM_REFUSED_BUDGET,
                  FramePipeline, KVTileManager, TileGatingPolicy, TileLayout,
                  attn_forward_frames, attn_forward_launcher, attn_forward_launcher_bf16,
                  attn_forward_range, attn_forward_single_frame, attn_forward_single_frame_bf16, attn_splits,
                  device_sync, make_policy, set_stream)

__all__ = [
    "BF16", "FP32", "HEAD_DIM", "KVTM_ADMITTED", "KVTM_INVALID", "KVTM_REFUSED_BUDGET",
    "CLI_PATH", "LIB_PATH", "PKG_ROOT", "LibraryMissing", "last_error", "load",
    "FramePipeline", "KVTileManager", "TileGatingPolicy", "TileLayout",
    "attn_forward_frames", "attn_forward_launcher", "attn_forward_launcher_bf16",
    "attn_forward_range",
    "attn_forward_single_frame", "attn_forward_single_frame_bf16", "attn_splits",
    "device_sync", "make_policy", "set_stream", "backbone",
]
