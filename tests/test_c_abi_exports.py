"""libkvpersist.so loads and exports every entry point include/*.h declares.

No compute is called here (no GPU needed): extern "C" functions of
kvp_c_api.h are resolved through ctypes; the C++-linkage API of
attn_kernel.h, kv_tile_manager.h and tile_gating_policy.h is checked in the
dynamic symbol table (demangled).
"""

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
INCLUDE = ROOT / "include"


def _c_api_names():
    text = "\n".join(p.read_text() for p in sorted(INCLUDE.glob("kvp_*.h")))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set()
    for m in re.finditer(r"^\s*[A-Za-z_][\w\s\*]*?\b(kv[a-z_0-9]+)\s*\(", text, flags=re.M):
        names.add(m.group(1))
    return sorted(names)


def test_every_c_symbol_is_exported(lib):
    names = _c_api_names()
    assert len(names) > 60
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_python_binding_covers_header():
    from kvpersist import _lib
    names = set(_c_api_names())
    assert names == set(_lib.SIGNATURES), sorted(names ^ set(_lib.SIGNATURES))


def _dynamic_symbols():
    nm = shutil.which("nm")
    if nm is None:
        pytest.skip("nm not available")
    from kvpersist import _lib
    out = subprocess.run([nm, "-DC", "--defined-only", str(_lib.LIB_PATH)], check=True,
                         capture_output=True, text=True).stdout
    return out


def test_cpp_api_symbols_exported():
    syms = _dynamic_symbols()
    wanted = [
        "attn_forward_launcher(float const*, float const*, float const*, float const*, "
        "long const*, float*, int, int, int, int, bool)",
        "attn_forward_single_frame(float const*, float const*, float const*, float const*, "
        "long const*, float*, int, int, int, int, int)",
        "KVTileManager::KVTileManager(unsigned long, unsigned long)",
        "KVTileManager::init()",
        "KVTileManager::admit(long, void*, unsigned long)",
        "KVTileManager::release(long)",
        "KVTileManager::clear()",
        "KVTileManager::persisted_tiles() const",
        "KVTileManager::is_persisted(long) const",
        "KVTileManager::query_device_limit() const",
        "KVTileManager::arena_init(unsigned long, unsigned long)",
        "KVTileManager::arena_begin_step()",
        "KVTileManager::arena_stage(void const*, unsigned long, void const*, unsigned long, long*)",
        "KVTileManager::arena_apply_window()",
        "KVTileManager::arena_end_step()",
        "KVTileManager::arena_device_ptr() const",
        "KVTileManager::streaming_begin()",
        "KVTileManager::streaming_stage(long, void const*, unsigned long, void const*, "
        "unsigned long, bool, long*, bool*)",
        "KVTileManager::streaming_release(long)",
        "KVTileManager::streaming_apply_window()",
        "KVTileManager::streaming_end()",
        "NoPersistencePolicy::select(float const*, int, int, long*, int*)",
        "UniformWindowPolicy::select(float const*, int, int, long*, int*)",
        "RecencyWindowPolicy::select(float const*, int, int, long*, int*)",
        "ReuseWeightedPolicy::ReuseWeightedPolicy(int, int)",
        "ReuseWeightedPolicy::select(float const*, int, int, long*, int*)",
        "MotionGatedPolicy::select(float const*, int, int, long*, int*)",
        "make_tile_gating_policy(char const*, int, int)",
    ]
    missing = [w for w in wanted if w not in syms]
    assert not missing, missing


def test_policy_names(lib):
    for name in ("none", "uniform", "recency", "motion", "reuse_weighted"):
        p = lib.kvp_policy_create(name.encode(), 98, 8)
        assert p
        assert lib.kvp_policy_name(p).decode() == name
        lib.kvp_policy_destroy(p)
    assert not lib.kvp_policy_create(b"bogus", 98, 8)


def test_attention_rejects_bad_shapes_without_touching_device(lib):
    # head_dim != 128 is refused before any device call
    rc = lib.kvp_attn_forward_range(0, 16, 16, 16, None, None, 16, 10, 100, 1, 0, 10, None)
    assert rc != 0 and b"head_dim" in lib.kvp_last_error()
    rc = lib.kvp_attn_forward_range(0, 16, 16, 16, None, None, 16, 10, 128, 1, 5, 5, None)
    assert rc != 0 and b"key range" in lib.kvp_last_error()
    rc = lib.kvp_attn_forward_range(7, 16, 16, 16, None, None, 16, 10, 128, 1, 0, 5, None)
    assert rc != 0 and b"dtype" in lib.kvp_last_error()
