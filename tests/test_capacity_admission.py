"""Capacity/admission scenario S1-S8 through the C-ABI facade (kvtm_*).

Mirrors the reference test step for step (reference:
tests/test_capacity_admission.py:63-154) with the budget numbers of its
grounding config: 22 tiles of 98,304 B fill 2,162,688 B exactly, tile 23 is
refused, duplicates never double-count, release frees room, clear resets,
and the tile layout of 1560 tokens gives 98 tiles with a last count of 8.

Admission is pure host bookkeeping, so the scenario runs without a GPU on
host-only addresses (never dereferenced), and again, marked gpu, on tiles
carved from kvtm_dev_alloc memory, as in the reference.
"""

import ctypes
import json
from pathlib import Path

import pytest

OK, REFUSED, INVALID = 1, 0, -1
META = json.loads((Path(__file__).parent / "golden" / "reference_meta.json").read_text())


def _scratch(lib, nbytes, on_device):
    if on_device:
        p = lib.kvtm_dev_alloc(nbytes)
        assert p, "scratch alloc failed"
        return p, True
    return 0x7F0000000000, False  # host-only: the manager never dereferences it


def test_capacity_admission(lib):
    _scenario(lib, on_device=False)


@pytest.mark.gpu
def test_capacity_admission_on_device_memory(lib):
    assert lib.kvp_device_count() > 0
    _scenario(lib, on_device=True)


def _scenario(lib, on_device):
    g = META["grounding"]
    budget, tile_bytes = g["max_persisting_l2_bytes"], g["kv_tile_bytes"]
    expected = g["tiles_fully_persistable"]
    max_window = g["access_policy_max_window_bytes"]
    tpf, tt = g["tokens_per_frame"], g["tile_size_tokens"]
    assert budget % tile_bytes == 0 and budget // tile_bytes == expected

    m = lib.kvtm_create(budget, max_window)
    assert m
    scratch, on_device = _scratch(lib, budget + 4 * tile_bytes, on_device)
    try:
        # S1: init + read-back of the configured limit
        assert lib.kvtm_init(m) == 1
        assert lib.kvtm_query_limit(m) == budget

        def admit(i):
            return lib.kvtm_admit(m, i, ctypes.c_void_p(scratch + i * tile_bytes), tile_bytes)

        # S2: exact fill
        assert [admit(i) for i in range(expected)] == [OK] * expected
        assert lib.kvtm_persisted_bytes(m) == expected * tile_bytes == budget
        assert lib.kvtm_persisted_tiles(m) == expected
        # S3: overflow refused, nothing counted
        assert admit(expected) == REFUSED
        assert lib.kvtm_persisted_bytes(m) == budget
        # S4: duplicate admit invalid, no double count
        assert admit(5) == INVALID
        assert lib.kvtm_persisted_tiles(m) == expected
        assert lib.kvtm_persisted_bytes(m) == budget
        # S5: release frees exactly one tile; double release rejected
        assert lib.kvtm_release(m, 7) == 1
        assert lib.kvtm_persisted_bytes(m) == budget - tile_bytes
        assert lib.kvtm_release(m, 7) == 0
        # S6: freed room reused, next candidate refused again
        assert admit(expected) == OK
        assert lib.kvtm_persisted_tiles(m) == expected
        assert admit(expected + 1) == REFUSED
        # S7: clear resets, admit works again
        lib.kvtm_clear(m)
        assert lib.kvtm_persisted_tiles(m) == 0
        assert lib.kvtm_persisted_bytes(m) == 0
        assert admit(90) == OK
        # S8: tile layout
        tiles = lib.kvtm_layout_tiles_per_frame(tpf, tt)
        assert tiles == (tpf + tt - 1) // tt == 98
        counts = []
        for i in range(tiles):
            s = lib.kvtm_layout_tile_start(tpf, tt, i)
            c = lib.kvtm_layout_tile_count(tpf, tt, i)
            assert s == i * tt and c == min(tt, tpf - s)
            counts.append(c)
        assert sum(counts) == tpf == 1560 and counts[-1] == 8
    finally:
        if on_device:
            lib.kvtm_dev_free(ctypes.c_void_p(scratch))
        lib.kvtm_destroy(m)


def test_admit_argument_checks(lib):
    m = lib.kvtm_create(1000, 500)
    try:
        p = ctypes.c_void_p(0x1000)
        assert lib.kvtm_admit(m, 0, p, 10) == INVALID          # before init
        assert lib.kvtm_init(m) == 1
        assert lib.kvtm_admit(m, -1, p, 10) == INVALID
        assert lib.kvtm_admit(m, 0, None, 10) == INVALID
        assert lib.kvtm_admit(m, 0, p, 0) == INVALID
        assert lib.kvtm_admit(m, 0, p, 501) == INVALID         # above max window
        assert lib.kvtm_admit(m, 0, p, 500) == OK
        assert lib.kvtm_is_persisted(m, 0) == 1
        assert lib.kvtm_admit(m, 1, p, 500) == OK
        assert lib.kvtm_admit(m, 2, p, 1) == REFUSED
        assert lib.kvtm_release(m, 3) == 0
    finally:
        lib.kvtm_destroy(m)


def test_init_refuses_budget_above_residency_limit(lib):
    m = lib.kvtm_create((256 << 20) + 1, 1 << 30)
    try:
        assert lib.kvtm_init(m) == 0
        assert lib.kvtm_query_limit(m) == 0
    finally:
        lib.kvtm_destroy(m)
