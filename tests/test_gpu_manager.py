"""KVTileManager per-row API with real device copies.

The reference issues two cudaMemcpyAsync per staged row; here stage calls
record copies that one gather launch executes at the next flush point. The
arena contents after a flush must be exactly what the reference's copies
would have produced.
"""

import numpy as np
import pytest
import torch

from kvpersist import KVTileManager

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rows(n, D, seed, dtype=torch.float32):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(n, D, generator=g).to(dtype).to(DEV)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_arena_stage_rows_land_in_order(dtype):
    D = 256
    esz = 4 if dtype == torch.float32 else 2
    K, V = _rows(50, D, 1, dtype), _rows(50, D, 2, dtype)
    row_bytes = D * esz
    stride_floats = 2 * D * esz // 4
    cap = 20 * 2 * row_bytes
    m = KVTileManager(cap, cap)
    assert m.init() and m.arena_init(cap, stride_floats)
    m.arena_begin_step()
    src = [7, 3, 42, 0, 19, 19]
    rows = [m.arena_stage(K[r].data_ptr(), row_bytes, V[r].data_ptr(), row_bytes) for r in src]
    assert rows == list(range(len(src)))
    assert m.pending_copies() == len(src)
    assert m.arena_apply_window()
    assert m.pending_copies() == 0
    arena = torch.empty(20, 2 * D, dtype=dtype, device=DEV)
    torch.cuda.synchronize()
    from kvpersist import _lib
    assert _lib.load().kvp_memcpy_d2d(arena.data_ptr(), m.arena_device_ptr(),
                                      arena.numel() * esz, None) == 0
    torch.cuda.synchronize()
    for i, r in enumerate(src):
        assert torch.equal(arena[i, :D], K[r]) and torch.equal(arena[i, D:], V[r])
    m.arena_end_step()
    m.close()


def test_streaming_restage_and_slot_reuse_last_copy_wins():
    D = 128
    K, V = _rows(10, D, 3), _rows(10, D, 4)
    rb = D * 4
    cap = 4 * 2 * rb
    m = KVTileManager(cap, cap)
    assert m.init() and m.arena_init(cap, 2 * D)
    assert m.streaming_begin()
    ok, s5, re = m.streaming_stage(5, K[5].data_ptr(), rb, V[5].data_ptr(), rb)
    assert ok and s5 == 0 and re
    assert m.streaming_apply_window()
    K[5] += 1.0  # content changed on the device: restage with changed=True
    ok, s, re = m.streaming_stage(5, K[5].data_ptr(), rb, V[5].data_ptr(), rb, changed=True)
    assert ok and s == 0 and re
    ok, s, re = m.streaming_stage(5, K[5].data_ptr(), rb, V[5].data_ptr(), rb)
    assert ok and s == 0 and not re      # sticky hit: nothing recorded
    # slot reuse inside one step: stage 6 -> slot 1, release, stage 7 -> slot 1
    ok, s6, _ = m.streaming_stage(6, K[6].data_ptr(), rb, V[6].data_ptr(), rb)
    assert s6 == 1 and m.streaming_release(6)
    ok, s7, _ = m.streaming_stage(7, K[7].data_ptr(), rb, V[7].data_ptr(), rb)
    assert s7 == 1
    assert m.pending_copies() == 2       # slot 0 (restage) + slot 1 (row 7 only)
    assert m.flush()
    arena = torch.empty(4, 2 * D, device=DEV)
    from kvpersist import _lib
    torch.cuda.synchronize()
    assert _lib.load().kvp_memcpy_d2d(arena.data_ptr(), m.arena_device_ptr(),
                                      arena.numel() * 4, None) == 0
    torch.cuda.synchronize()
    assert torch.equal(arena[0, :D], K[5]) and torch.equal(arena[0, D:], V[5])
    assert torch.equal(arena[1, :D], K[7]) and torch.equal(arena[1, D:], V[7])
    assert m.streaming_staged_bytes() == 4 * 2 * rb
    m.streaming_end()
    m.close()


def test_attached_arena_is_used_in_place():
    D = 128
    K, V = _rows(4, D, 5), _rows(4, D, 6)
    rb = D * 4
    buf = torch.zeros(8, 2 * D, device=DEV)
    m = KVTileManager(buf.numel() * 4, buf.numel() * 4)
    assert m.init() and m.arena_attach(buf, buf.numel() * 4, 2 * D)
    m.arena_begin_step()
    assert m.arena_stage(K[2].data_ptr(), rb, V[2].data_ptr(), rb) == 0
    assert m.flush()
    torch.cuda.synchronize()
    assert torch.equal(buf[0, :D], K[2]) and torch.equal(buf[0, D:], V[2])
    assert int(buf[1:].abs().sum()) == 0
    m.close()
    torch.cuda.synchronize()
    assert torch.equal(buf[0, :D], K[2])  # caller-owned memory outlives the manager
