"""kvp_stage_run: one flush = arena row copies + KVMap entries in one launch.

A flush whose copies and map entries form few runs (consecutive source rows
to consecutive arena rows; consecutive map rows with consecutive slots, or
resets to -1) travels as kernel arguments; any other flush reads its
descriptors from mapped host memory. Both encodings must leave exactly the
bytes the reference's per-row copies (src/kv_tile_manager.cu:104-121) and its
host-built KVMap upload would leave.
"""

import ctypes

import numpy as np
import pytest
import torch

from kvpersist import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


class KvpRowCopy(ctypes.Structure):
    _fields_ = [("k_src", ctypes.c_void_p), ("v_src", ctypes.c_void_p),
                ("dst_row", ctypes.c_long), ("k_bytes", ctypes.c_uint), ("v_bytes", ctypes.c_uint)]


def _flush(lib, stager, arena, stride, K, V, src_rows, dst_rows, map_dev, m_rows, m_slots):
    esz = K.element_size()
    kb = K.shape[1] * esz
    n = len(src_rows)
    arr = (KvpRowCopy * max(1, n))()
    for i, (s, d) in enumerate(zip(src_rows, dst_rows)):
        arr[i] = KvpRowCopy(K.data_ptr() + s * kb, V.data_ptr() + s * kb, d, kb, kb)
    mr = np.asarray(m_rows, dtype=np.int64)
    ms = np.asarray(m_slots, dtype=np.int64)
    rc = lib.kvp_stage_run(stager, arena.data_ptr(), stride, ctypes.cast(arr, ctypes.c_void_p), n,
                           map_dev.data_ptr() if map_dev is not None else None, 0,
                           mr.ctypes.data if len(mr) else None, ms.ctypes.data if len(ms) else None,
                           len(mr), None)
    assert rc == 0, lib.kvp_last_error()


def _expect(arena_rows, D, K, V, src_rows, dst_rows):
    exp = arena_rows.clone()
    for s, d in zip(src_rows, dst_rows):
        exp[d, :D] = K[s]
        exp[d, D:] = V[s]
    return exp


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("pattern", ["runs", "scattered"])
def test_stage_run_copies_and_map(dtype, pattern):
    lib = _lib.load()
    D, N, A = 384, 2000, 900
    g = torch.Generator(device="cpu").manual_seed(11)
    K = torch.randn(N, D, generator=g).to(dtype).to(DEV)
    V = torch.randn(N, D, generator=g).to(dtype).to(DEV)
    arena = torch.randn(A, 2 * D, generator=g).to(dtype).to(DEV)
    kvmap = torch.full((N,), -7, dtype=torch.long, device=DEV)
    stride = 2 * D * K.element_size()
    rng = np.random.default_rng(5)
    if pattern == "runs":
        # 20 tiles of 16 rows, consecutive arena rows per tile: 20 copy runs
        tiles = rng.choice(N // 16, size=20, replace=False)
        src = [int(t) * 16 + r for t in tiles for r in range(16)]
        dst = list(range(100, 100 + len(src)))
        m_rows = src + list(range(1500, 1540))
        m_slots = dst + [-1] * 40
    else:
        src = [int(x) for x in rng.choice(N, size=300, replace=False)]
        dst = [int(x) for x in rng.choice(A, size=300, replace=False)]
        m_rows = src
        m_slots = dst
    stager = lib.kvp_stager_create()
    try:
        before = arena.clone()
        _flush(lib, stager, arena, stride, K, V, src, dst, kvmap, m_rows, m_slots)
        torch.cuda.synchronize()
        assert torch.equal(arena, _expect(before, D, K, V, src, dst))
        exp_map = torch.full((N,), -7, dtype=torch.long)
        exp_map[torch.tensor(m_rows)] = torch.tensor(m_slots)
        assert torch.equal(kvmap.cpu(), exp_map)
        # a second flush on the same stager: copies only, then map only
        src2, dst2 = src[:5], [0, 1, 2, 3, 4]
        _flush(lib, stager, arena, stride, K, V, src2, dst2, None, [], [])
        _flush(lib, stager, arena, stride, K, V, [], [], kvmap, [3, 4, 5], [9, 10, 11])
        torch.cuda.synchronize()
        exp2 = _expect(before, D, K, V, src, dst)
        exp2 = _expect(exp2, D, K, V, src2, dst2)
        assert torch.equal(arena, exp2)
        exp_map[torch.tensor([3, 4, 5])] = torch.tensor([9, 10, 11])
        assert torch.equal(kvmap.cpu(), exp_map)
    finally:
        lib.kvp_stager_destroy(stager)


def test_stage_run_unaligned_rows_use_byte_copies():
    lib = _lib.load()
    D, N = 37, 64   # 37 fp32 = 148-byte rows: not a multiple of 16
    g = torch.Generator(device="cpu").manual_seed(2)
    K = torch.randn(N, D, generator=g).to(DEV)
    V = torch.randn(N, D, generator=g).to(DEV)
    arena = torch.zeros(16, 2 * D, device=DEV)
    stager = lib.kvp_stager_create()
    try:
        src, dst = [10, 11, 12, 40], [3, 4, 5, 0]
        _flush(lib, stager, arena, 2 * D * 4, K, V, src, dst, None, [], [])
        torch.cuda.synchronize()
        assert torch.equal(arena, _expect(torch.zeros(16, 2 * D, device=DEV), D, K, V, src, dst))
    finally:
        lib.kvp_stager_destroy(stager)


def test_stage_ring_wraps_and_changes_stream_without_host_waits():
    """120 descriptor-ring flushes of ~96 KB each (the 4 MiB ring wraps twice),
    issued back to back with no host synchronisation, the first 60 on
    one stream and the rest on another: the ring reuses a region only after
    the launches that read it have finished, and a change of stream waits
    for the earlier one, so the arena and the KVMap end as a sequential
    replay of the flushes leaves them."""
    lib = _lib.load()
    D, N, A, n = 256, 4096, 4096, 2000
    dtype = torch.bfloat16
    g = torch.Generator(device="cpu").manual_seed(21)
    K = torch.randn(N, D, generator=g).to(dtype)
    V = torch.randn(N, D, generator=g).to(dtype)
    Kd, Vd = K.to(DEV), V.to(DEV)
    arena = torch.zeros(A, 2 * D, dtype=dtype, device=DEV)
    kvmap = torch.full((N,), -1, dtype=torch.long, device=DEV)
    exp_arena = torch.zeros(A, 2 * D, dtype=dtype)
    exp_map = torch.full((N,), -1, dtype=torch.long)
    kb = D * K.element_size()
    stride = 2 * kb
    rng = np.random.default_rng(8)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    keep = []  # host descriptor arrays stay alive until the end
    stager = lib.kvp_stager_create()
    try:
        for i in range(120):
            src = rng.choice(N, size=n, replace=True)
            dst = rng.choice(A, size=n, replace=False)
            arr = (KvpRowCopy * n)()
            for j in range(n):
                arr[j] = KvpRowCopy(Kd.data_ptr() + int(src[j]) * kb,
                                    Vd.data_ptr() + int(src[j]) * kb, int(dst[j]), kb, kb)
            mr = rng.choice(N, size=n, replace=False).astype(np.int64)
            ms = rng.integers(-1, A, size=n).astype(np.int64)
            keep.append((arr, mr, ms))
            st = streams[0 if i < 60 else 1]
            rc = lib.kvp_stage_run(stager, arena.data_ptr(), stride, ctypes.cast(arr, ctypes.c_void_p),
                                   n, kvmap.data_ptr(), 0, mr.ctypes.data, ms.ctypes.data, n,
                                   ctypes.c_void_p(st.cuda_stream))
            assert rc == 0, lib.kvp_last_error()
            exp_arena[torch.from_numpy(dst)] = torch.cat([K[torch.from_numpy(src)],
                                                          V[torch.from_numpy(src)]], dim=1)
            exp_map[torch.from_numpy(mr)] = torch.from_numpy(ms)
        torch.cuda.synchronize()
        assert torch.equal(arena.cpu(), exp_arena)
        assert torch.equal(kvmap.cpu(), exp_map)
    finally:
        lib.kvp_stager_destroy(stager)
