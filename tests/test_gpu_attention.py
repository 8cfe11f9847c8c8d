"""GPU parity of the attention kernels against the CPU oracle.

Tolerances: fp32 max-abs <= 1e-3 and mean-abs <= 1e-4
against the fp32 golden (reference: tests/test_correctness.py:26-27);
bf16 max-abs <= 2e-2 against the fp32 golden of bf16-rounded inputs.
KVMap indirection must not change a single bit of the output.
"""

import numpy as np
import pytest
import torch

from kvpersist import api, workloads
from oracle import attention as at
from oracle import trace_synth as ts

pytestmark = pytest.mark.gpu
DEV = "cuda"
FP32_MAX, FP32_MEAN, BF16_MAX = 1e-3, 1e-4, 2e-2


def _inputs(frames, T, heads, seed, dtype):
    rng = np.random.default_rng(seed)
    D = heads * 128
    q, k, v = (torch.from_numpy(rng.standard_normal((frames * T, D), dtype=np.float32))
               for _ in range(3))
    if dtype == torch.bfloat16:
        q, k, v = at.round_bf16(q), at.round_bf16(k), at.round_bf16(v)
    return q, k, v


def _run(dtype, q, k, v, frames, T, heads, mode, window=0, arena=None, kvmap=None):
    """Per-frame launches through the C-ABI (intra: pre-offset; cross: full bases)."""
    D = heads * 128
    qd, kd, vd = (x.to(DEV).to(dtype).contiguous() for x in (q, k, v))
    out = torch.empty_like(qd)
    for f in range(frames):
        sl = slice(f * T, (f + 1) * T)
        if mode == "intra":
            kv_k, kv_v = kd[sl], vd[sl]
            mp = kvmap[sl] if kvmap is not None else None
        else:
            kv_k, kv_v, mp = kd, vd, kvmap
        if dtype == torch.float32:
            api.attn_forward_single_frame(qd[sl], kv_k, kv_v, arena, mp, out[sl], T, D, heads,
                                          0 if mode == "intra" else 1, f, window)
        else:
            api.attn_forward_single_frame_bf16(qd[sl], kv_k, kv_v, arena, mp, out[sl], T, D,
                                               heads, 0 if mode == "intra" else 1, f, window)
    torch.cuda.synchronize()
    return out.float().cpu()


def _check(got, want, dtype):
    err = (got - want).abs()
    if dtype == torch.float32:
        assert float(err.max()) <= FP32_MAX, float(err.max())
        assert float(err.mean()) <= FP32_MEAN, float(err.mean())
    else:
        assert float(err.max()) <= BF16_MAX, float(err.max())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode,window", [("intra", 0), ("cross", 0), ("cross", 2)])
@pytest.mark.parametrize("T,heads", [(200, 2), (33, 1), (1, 1), (129, 3)])
def test_small_shapes_match_oracle(dtype, mode, window, T, heads):
    frames = 4
    q, k, v = _inputs(frames, T, heads, seed=T * 7 + heads, dtype=dtype)
    got = _run(dtype, q, k, v, frames, T, heads, mode, window)
    want = at.attention_frames(q, k, v, frames, T, heads, mode, window)
    _check(got, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_single_key_returns_value_row_exactly(dtype):
    q, k, v = _inputs(1, 1, 2, seed=3, dtype=dtype)
    got = _run(dtype, q, k, v, 1, 1, 2, "intra")
    assert torch.equal(got, v.to(dtype).float())


def _random_arena(k, v, rng, frac=0.3):
    """Copy a random subset of K|V rows to permuted arena rows; return arena, map."""
    rows = k.shape[0]
    D = k.shape[1]
    chosen = rng.choice(rows, size=max(1, int(frac * rows)), replace=False)
    slots = rng.permutation(len(chosen))
    arena = torch.zeros(len(chosen) + 3, 2 * D, dtype=k.dtype)
    kvmap = torch.full((rows,), -1, dtype=torch.int64)
    for r, s in zip(chosen, slots):
        arena[s, :D] = k[r]
        arena[s, D:] = v[r]
        kvmap[r] = int(s)
    return arena, kvmap


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["intra", "cross"])
def test_kvmap_indirection_is_bitwise_invisible(dtype, mode):
    frames, T, heads = 3, 300, 2
    q, k, v = _inputs(frames, T, heads, seed=11, dtype=dtype)
    base = _run(dtype, q, k, v, frames, T, heads, mode)
    rng = np.random.default_rng(12)
    arena, kvmap = _random_arena(k.to(dtype), v.to(dtype), rng)
    got = _run(dtype, q, k, v, frames, T, heads, mode, arena=arena.to(DEV).contiguous(),
               kvmap=kvmap.to(DEV))
    assert torch.equal(got, base)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kvmap_with_key_splits_is_bitwise_invisible(dtype):
    """Cross-frame shape that splits the key range (several tiles per split, a
    partial last tile): the KVMap launch equals the map-free launch bit for bit,
    and both match the oracle."""
    frames, T, heads = 2, 1560, 12
    d = 1 if dtype == torch.bfloat16 else 0
    assert api.attn_splits(d, T, heads, 1, frames * T) > 1
    q, k, v = _inputs(frames, T, heads, seed=13, dtype=dtype)
    base = _run(dtype, q, k, v, frames, T, heads, "cross")
    rng = np.random.default_rng(14)
    arena, kvmap = _random_arena(k.to(dtype), v.to(dtype), rng, frac=0.25)
    got = _run(dtype, q, k, v, frames, T, heads, "cross", arena=arena.to(DEV).contiguous(),
               kvmap=kvmap.to(DEV))
    assert torch.equal(got, base)
    _check(base, at.attention_frames(q, k, v, frames, T, heads, "cross"), dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kvmap_group_shapes_bitwise_invisible(dtype):
    """The bf16 kernel copies a 16-row group whose rows all map to
    consecutive arena rows (a run) like an unmapped group, from the arena;
    every other mapped group chooses each row's source per lane. Groups of
    every shape the run check tells apart — unmapped, run, run from arena
    row 0, reversed, a run with one hole (row 5, or row 0), a jump between
    two halves, a jump at a 4-row boundary, and a partial last group — must
    give the map-free output bit for bit; arena rows no entry names hold
    NaN, so a wrong read would show."""
    frames, T, heads = 1, 680, 2
    D = heads * 128
    q, k, v = _inputs(frames, T, heads, seed=21, dtype=dtype)
    base = _run(dtype, q, k, v, frames, T, heads, "cross")
    kvmap = torch.full((T,), -1, dtype=torch.int64)
    nxt = 16  # arena rows 0..15 belong to the first run based at row 0
    zero_used = False
    for g in range((T + 15) // 16):
        rows = list(range(16 * g, min(16 * g + 16, T)))
        n, pat = len(rows), g % 8
        if pat == 0:
            continue
        if pat == 7 and not zero_used:
            b, zero_used = 0, True
        else:
            b = nxt
            nxt += n + 128
        slots = [b + j for j in range(n)]
        if pat == 2:
            slots = slots[::-1]
        elif pat == 3 and n > 5:
            slots[5] = -1
        elif pat == 4:
            slots[0] = -1
        elif pat == 5:
            slots = [b + j + (50 if j >= 8 else 0) for j in range(n)]
        elif pat == 6:
            slots = [b + j + (100 if j >= 4 else 0) for j in range(n)]
        for r, s in zip(rows, slots):
            kvmap[r] = s
    arena = torch.full((nxt, 2 * D), float("nan"), dtype=dtype)
    kt, vt = k.to(dtype), v.to(dtype)
    for r in range(T):
        s = int(kvmap[r])
        if s >= 0:
            arena[s, :D] = kt[r]
            arena[s, D:] = vt[r]
    got = _run(dtype, q, k, v, frames, T, heads, "cross", arena=arena.to(DEV).contiguous(),
               kvmap=kvmap.to(DEV))
    assert torch.equal(got, base)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kvmap_entries_outside_arena_rows_read_original(dtype):
    """Negative entries of any value read the original K/V row, valid entries
    their arena row. bf16 also: entries whose arena row would end beyond the
    arena's first 4 GiB (2*(m+1)*row_bytes > 2^32) read the original row; the
    fp32 kernel indexes the arena with any m >= 0, as the reference does, so
    such entries are not given to it."""
    frames, T, heads = 1, 700, 2
    q, k, v = _inputs(frames, T, heads, seed=15, dtype=dtype)
    base = _run(dtype, q, k, v, frames, T, heads, "cross")
    rng = np.random.default_rng(16)
    arena, kvmap = _random_arena(k.to(dtype), v.to(dtype), rng, frac=0.2)
    odd = torch.from_numpy(rng.choice(T, size=200, replace=False))
    vals = [-2, -7, -(1 << 40), -(1 << 63)]
    if dtype == torch.bfloat16:
        row_bytes = heads * 128 * 2
        vals += [(1 << 31) // row_bytes, 1 << 31, (1 << 31) + 5, 1 << 40, 1 << 62]
    specials = torch.tensor(vals, dtype=torch.int64)
    kvmap[odd] = specials[torch.arange(200) % len(specials)]
    got = _run(dtype, q, k, v, frames, T, heads, "cross", arena=arena.to(DEV).contiguous(),
               kvmap=kvmap.to(DEV))
    assert torch.equal(got, base)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_c1_full_frame(dtype):
    """C1 shape: 1560 tokens x 12 heads x 128, policy none."""
    T, heads = 1560, 12
    q, k, v = (torch.from_numpy(x) for x in workloads.qkv_host(1, T, seed=42))
    if dtype == torch.bfloat16:
        q, k, v = at.round_bf16(q), at.round_bf16(k), at.round_bf16(v)
    got = _run(dtype, q, k, v, 1, T, heads, "intra")
    _check(got, at.attention_keys(q, k, v, heads), dtype)


def test_reference_trace_baseline_launcher():
    """The reference correctness scoreboard: baseline launcher (remap=false,
    8 frames in one launch) on the reference's own seed-42 trace against the
    fp32 golden, max-abs < 1e-3 and mean-abs < 1e-4 per frame
    (reference: tests/test_correctness.py:26-27,86-97)."""
    torch.set_num_threads(min(16, max(1, torch.get_num_threads())))
    tr = ts.synthetic_trace(frames=8, seed=42)
    T, D, heads = 1560, 1536, 12
    q = tr["q"].reshape(-1, D).to(DEV)
    k = tr["k"].reshape(-1, D).to(DEV)
    v = tr["v"].reshape(-1, D).to(DEV)
    out = torch.empty_like(q)
    api.attn_forward_launcher(q, k, v, None, None, out, 8, T, D, heads, remap=False)
    torch.cuda.synchronize()
    got = out.cpu().view(8, T, D)
    for f in range(8):
        want = at.attention_keys(tr["q"][f], tr["k"][f], tr["v"][f], heads)
        err = (got[f] - want).abs()
        assert float(err.max()) < FP32_MAX and float(err.mean()) < FP32_MEAN, f


def test_launcher_remap_equals_baseline():
    frames, T, heads = 3, 257, 2
    q, k, v = _inputs(frames, T, heads, seed=21, dtype=torch.float32)
    D = heads * 128
    rng = np.random.default_rng(22)
    arena, kvmap_abs = _random_arena(k, v, rng, frac=0.4)
    # remap=true slices the map per frame: map[f*T + j] for key j of frame f
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    out_a = torch.empty_like(qd)
    out_b = torch.empty_like(qd)
    api.attn_forward_launcher(qd, kd, vd, None, None, out_a, frames, T, D, heads, remap=False)
    api.attn_forward_launcher(qd, kd, vd, arena.to(DEV), kvmap_abs.to(DEV), out_b, frames, T, D,
                              heads, remap=True)
    torch.cuda.synchronize()
    assert torch.equal(out_a.cpu(), out_b.cpu())
    want = at.attention_frames(q, k, v, frames, T, heads, "intra")
    _check(out_a.cpu(), want, torch.float32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_split_and_unsplit_launches(dtype):
    """One frame of 1560 queries splits the key range (grid underfill); a short
    key range (fewer than 8 key tiles) never does. Both paths must match the
    oracle."""
    T, heads = 1560, 12
    d = 1 if dtype == torch.bfloat16 else 0
    assert api.attn_splits(d, T, heads, 1, T) > 1
    assert api.attn_splits(d, 200, heads, 1, 200) == 1
    for t, frames in ((T, 2), (200, 3)):
        q, k, v = _inputs(frames, t, heads, seed=31, dtype=dtype)
        got = _run(dtype, q, k, v, frames, t, heads, "cross")
        want = at.attention_frames(q, k, v, frames, t, heads, "cross")
        _check(got, want, dtype)


def test_bad_arguments_are_rejected_before_launch(lib):
    x = torch.zeros(64, 256, device=DEV)
    # map without arena
    m = torch.zeros(64, dtype=torch.int64, device=DEV)
    rc = lib.kvp_attn_forward_range(0, x.data_ptr(), x.data_ptr(), x.data_ptr(), None,
                                    m.data_ptr(), x.data_ptr(), 64, 256, 2, 0, 64, None)
    assert rc != 0
    # misaligned pointer
    rc = lib.kvp_attn_forward_range(0, x.data_ptr() + 4, x.data_ptr(), x.data_ptr(), None, None,
                                    x.data_ptr(), 63, 256, 2, 0, 63, None)
    assert rc != 0
