"""GPU parity of the bf16 layer launch with group descriptors
(kvp_attn_forward_frames_gd), through the C-ABI.

The descriptor kernel reads one 8-byte entry per 16-row copy group and a
group's KVMap entries only when the entry says "general"; its output must
be bitwise that of the same launch reading the map alone
(kvp_attn_forward_frames), which keeps the reference's map semantics
(src/gated_attention_kernel.cu:73-85, :118-130):
* groups of every shape the descriptor tells apart (none, a full run, a
  run from arena row 0, half groups at rows 0-7 and 8-15, two sub-runs,
  three runs = general, reversed = general, a hole, a short last group)
  over an arena whose unnamed rows hold NaN, bitwise equal to the map-free
  launch, in causal, windowed (ranges starting 8 rows off the 16-row grid)
  and intra layers;
* arena rows holding other data than the rows they stand in for: the output
  equals the oracle's attention with those rows replaced, and the map-only
  launch bit for bit;
* a table of "general" entries only (every group decoded from the map);
* an empty table (every map entry -1, every descriptor "no arena row"):
  bitwise the map-free launch at the c3, c4 and c5 layer shapes, which is
  what lets bench.py time and count policy none through this kernel;
* the frame pipeline (kvp_pipeline_run, which writes the tables in its
  staging launch): device tables equal kvp_attn_group_desc over the device
  map slices after each of three layers, and the pipeline output equals
  the map-only launch over its arena and map bit for bit.
"""

import ctypes

import numpy as np
import pytest
import torch

from kvpersist import FramePipeline, _lib, api, workloads
from oracle import attention as at

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16_MAX = 2e-2


def _inputs(frames, T, heads, seed):
    rng = np.random.default_rng(seed)
    D = heads * 128
    return [at.round_bf16(torch.from_numpy(rng.standard_normal((frames * T, D),
                                                               dtype=np.float32)))
            for _ in range(3)]


def _ranges(mode, frames, T, window):
    return [at.key_range(mode, f, T, window) for f in range(frames)]


def _tables(kvmap, mode, frames, T, window, D, stride):
    """Descriptor tables of every frame's slice, [frames, gd_stride, 2]."""
    per = []
    for f, (b, e) in enumerate(_ranges(mode, frames, T, window)):
        sl = kvmap[f * stride:(f + 1) * stride].numpy()
        if mode == "intra":
            b, e = b - f * T, e - f * T
        per.append(api.attn_group_desc(sl, b, e, D))
    n = max(p.shape[0] for p in per)
    out = np.zeros((frames, n, 2), dtype=np.uint32)
    for f, p in enumerate(per):
        out[f, :p.shape[0]] = p
    return out


def _launch(qd, kd, vd, frames, T, heads, mode, window, arena=None, kvmap=None, stride=0,
            gd=None):
    out = torch.empty_like(qd)
    D = heads * 128
    if gd is None:
        api.attn_forward_frames(api.BF16, qd, kd, vd, arena, kvmap, out, frames, T, D, heads,
                                cross=(mode == "cross"), window_frames=window,
                                map_frame_stride=stride)
    else:
        gdd = torch.from_numpy(gd.view(np.int32)).to(DEV)
        api.attn_forward_frames_gd(qd, kd, vd, arena, kvmap, gdd, out, frames, T, D, heads,
                                   cross=(mode == "cross"), window_frames=window,
                                   map_frame_stride=stride, gd_frame_stride=gd.shape[1])
    torch.cuda.synchronize()
    return out


def _shaped_map(mode, frames, T, window, stride):
    """A KVMap whose groups cycle through every descriptor shape (per frame,
    groups relative to the frame's range start); arena rows handed out with
    gaps so that no two groups' rows touch."""
    kvmap = torch.full((frames * stride,), -1, dtype=torch.int64)
    nxt = 16  # arena rows 0..15: the run based at row 0
    zero_used = False
    for f, (b, e) in enumerate(_ranges(mode, frames, T, window)):
        rel = f * T if mode == "intra" else 0
        for g in range((e - b + 15) // 16):
            rows = list(range(b + 16 * g, min(b + 16 * g + 16, e)))
            n, pat = len(rows), (g + f) % 10
            if pat == 0:
                continue
            if pat == 9 and not zero_used:
                base, zero_used = 0, True
            else:
                base = nxt
                nxt += n + 64
            slots = [base + j for j in range(n)]
            if pat == 2:
                slots = slots[::-1]                      # general
            elif pat == 3:
                slots = [s if j < 8 else -1 for j, s in enumerate(slots)]   # rows 0-7
            elif pat == 4:
                slots = [s if j >= 8 else -1 for j, s in enumerate(slots)]  # rows 8-15
            elif pat == 5:
                slots = [base + j + (40 if j >= 8 else 0) for j in range(n)]  # two sub-runs
            elif pat == 6:
                slots = [base + j + (20 if j >= 4 else 0) + (20 if j >= 11 else 0)
                         for j in range(n)]              # three runs: general
            elif pat == 7 and n > 5:
                slots[5] = -1                            # hole: two sub-runs
            elif pat == 8:
                slots = [s if j % 2 else -1 for j, s in enumerate(slots)]  # general
            for r, s in zip(rows, slots):
                kvmap[f * stride + r - rel] = s
    return kvmap, nxt


@pytest.mark.parametrize("mode,window,T", [("cross", 0, 680), ("cross", 2, 680),
                                           ("cross", 2, 1000), ("intra", 0, 680)])
def test_descriptor_group_shapes_bitwise_invisible(mode, window, T):
    frames, heads = 4, 2
    D = heads * 128
    q, k, v = _inputs(frames, T, heads, seed=T + window)
    qd, kd, vd = (x.to(DEV).to(torch.bfloat16).contiguous() for x in (q, k, v))
    base = _launch(qd, kd, vd, frames, T, heads, mode, window)
    stride = frames * T if mode == "cross" else T
    kvmap, nrows = _shaped_map(mode, frames, T, window, stride)
    kt, vt = k.to(torch.bfloat16), v.to(torch.bfloat16)
    arena = torch.full((nrows, 2 * D), float("nan"), dtype=torch.bfloat16)
    for f in range(frames):
        for j in range(stride):
            s = int(kvmap[f * stride + j])
            if s >= 0:
                r = j + (f * T if mode == "intra" else 0)
                arena[s, :D], arena[s, D:] = kt[r], vt[r]
    gd = _tables(kvmap, mode, frames, T, window, D, stride)
    words = gd[:, :, 0]
    assert (words == 1).any() and (words == 0).any() and (words >= 0x80000000).any()
    assert (gd[:, :, 1] != 0).any(), "no two-sub-run group"
    ad, md = arena.to(DEV).contiguous(), kvmap.to(DEV)
    got_map = _launch(qd, kd, vd, frames, T, heads, mode, window, ad, md, stride)
    got_gd = _launch(qd, kd, vd, frames, T, heads, mode, window, ad, md, stride, gd)
    assert torch.equal(got_map, base)
    assert torch.equal(got_gd, base)


def test_descriptor_reads_the_arena_row_the_map_names():
    frames, T, heads = 3, 1560, 2
    D = heads * 128
    q, k, v = _inputs(frames, T, heads, seed=41)
    rng = np.random.default_rng(41)
    full = frames * T
    kvmap = torch.full((frames * full,), -1, dtype=torch.int64)
    n_arena = 0
    slots_of = []
    for f in range(frames):
        e = (f + 1) * T
        # tiles of 16 at the frame's own offsets (8 rows off the group grid
        # for odd frames), single rows, and the last partial tile
        tiles = rng.choice((e // 16) - 1, size=12, replace=False)
        rows = sorted({16 * int(t) + 8 * (f % 2) + j for t in tiles for j in range(16)}
                      | set(rng.choice(e, size=30, replace=False).tolist())
                      | set(range(e - 12, e)))
        rows = [r for r in rows if r < e]
        slots_of.append((rows, list(range(n_arena, n_arena + len(rows)))))
        n_arena += len(rows) + 32
    arena = at.round_bf16(torch.from_numpy(rng.standard_normal((n_arena, 2 * D),
                                                               dtype=np.float32)))
    want = torch.empty(frames * T, D)
    for f, (rows, slots) in enumerate(slots_of):
        e = (f + 1) * T
        kf, vf = k[:e].clone(), v[:e].clone()
        for r, s in zip(rows, slots):
            kvmap[f * full + r] = s
            kf[r], vf[r] = arena[s, :D], arena[s, D:]
        want[f * T:e] = at.attention_keys(q[f * T:e], kf, vf, heads)
    qd, kd, vd = (x.to(DEV).to(torch.bfloat16).contiguous() for x in (q, k, v))
    ad, md = arena.to(DEV).to(torch.bfloat16).contiguous(), kvmap.to(DEV)
    gd = _tables(kvmap, "cross", frames, T, 0, D, full)
    got_gd = _launch(qd, kd, vd, frames, T, heads, "cross", 0, ad, md, full, gd)
    got_map = _launch(qd, kd, vd, frames, T, heads, "cross", 0, ad, md, full)
    assert torch.equal(got_gd, got_map)
    err = float((got_gd.float().cpu() - want).abs().max())
    assert err <= BF16_MAX, err


def test_all_general_table_equals_map_launch():
    frames, T, heads = 3, 900, 1
    D = heads * 128
    q, k, v = _inputs(frames, T, heads, seed=5)
    rng = np.random.default_rng(5)
    full = frames * T
    kvmap = torch.full((frames * full,), -1, dtype=torch.int64)
    arena = at.round_bf16(torch.from_numpy(rng.standard_normal((4000, 2 * D),
                                                               dtype=np.float32)))
    for f in range(frames):
        e = (f + 1) * T
        rows = rng.choice(e, size=min(e, 500), replace=False)
        kvmap[f * full + torch.from_numpy(rows)] = torch.from_numpy(
            rng.choice(4000, size=rows.size, replace=False))
    gd = np.zeros((frames, 4 * ((full + 63) // 64), 2), dtype=np.uint32)
    gd[:, :, 0] = 1
    qd, kd, vd = (x.to(DEV).to(torch.bfloat16).contiguous() for x in (q, k, v))
    ad, md = arena.to(DEV).to(torch.bfloat16).contiguous(), kvmap.to(DEV)
    got_gd = _launch(qd, kd, vd, frames, T, heads, "cross", 0, ad, md, full, gd)
    got_map = _launch(qd, kd, vd, frames, T, heads, "cross", 0, ad, md, full)
    assert torch.equal(got_gd, got_map)


@pytest.mark.parametrize("frames,T,window", [(8, 1560, 0), (12, 1560, 8), (21, 3600, 0)])
def test_empty_table_equals_map_free_launch(frames, T, window):
    """Policy none through the descriptor launch (every map entry -1, every
    descriptor entry "no arena row", a one-row arena never read) is bitwise
    the map-free launch, at the layer shapes of the c3, c4 (fewer frames,
    same window) and c5 workloads."""
    print(f"empty table frames={frames} T={T} window={window}", flush=True)
    heads = workloads.HEADS
    D = workloads.HIDDEN
    q, k, v = workloads.qkv_device(frames, T, seed=frames + window, dtype=torch.bfloat16)
    span = frames * T
    longest = (min(window, frames) if window else frames) * T
    n = 4 * ((longest + 63) // 64)
    kvmap = torch.full((frames * span,), -1, dtype=torch.int64, device=DEV)
    gd = np.zeros((frames, n, 2), dtype=np.uint32)
    arena = torch.zeros((1, 2 * D), dtype=torch.bfloat16, device=DEV)
    free = _launch(q, k, v, frames, T, heads, "cross", window)
    empty = _launch(q, k, v, frames, T, heads, "cross", window, arena, kvmap, span, gd)
    assert torch.equal(free, empty)
    assert bool(torch.isfinite(free).all())


def _d2h(ptr, nbytes):
    buf = (ctypes.c_uint8 * nbytes)()
    assert _lib.load().kvp_memcpy_d2h(ctypes.addressof(buf), ptr, nbytes, None) == 0
    return np.frombuffer(bytes(buf), dtype=np.uint8)


@pytest.mark.parametrize("cfg_name,policy,streaming", [("c3", "motion", False),
                                                       ("c3", "recency", True),
                                                       ("c4", "reuse_weighted", False)])
def test_pipeline_tables_and_output(cfg_name, policy, streaming):
    cfg = workloads.CONFIGS[cfg_name]
    frames = min(cfg.frames, 10)
    T, D, H = cfg.tokens, workloads.HIDDEN, workloads.HEADS
    window = cfg.window
    pl = FramePipeline(policy, cross=True, streaming=streaming, frames=frames, T=T, D=D,
                       heads=H, tile_tokens=workloads.TILE_TOKENS, set_aside_bytes=cfg.set_aside,
                       dtype=api.BF16, window_frames=window)
    try:
        for layer in range(3):
            q, k, v = workloads.qkv_device(frames, T, seed=70 + layer, dtype=torch.bfloat16,
                                           device=DEV)
            out = torch.empty_like(q)
            pl.set_scores(workloads.motion_for(cfg, layer)[:frames])
            pl.run(q, k, v, out)
            torch.cuda.synchronize()
            stride, gstride = pl.layer_map_stride(), pl.layer_gd_stride()
            kvmap = _d2h(pl.layer_map_ptr(), frames * stride * 8).view(np.int64)
            gd = _d2h(pl.layer_gd_ptr(), frames * gstride * 8).view(np.uint32)
            gd = gd.reshape(frames, gstride, 2)
            want = _tables(torch.from_numpy(kvmap.copy()), "cross", frames, T, window, D, stride)
            np.testing.assert_array_equal(gd[:, :want.shape[1]], want, err_msg=f"layer {layer}")
            assert (gd[:, want.shape[1]:] == 0).all()
            assert (want[:, :, 0] >= 0x80000000).any()
            ref = torch.empty_like(q)
            api.attn_forward_frames(api.BF16, q, k, v, pl.layer_arena_ptr(), pl.layer_map_ptr(),
                                    ref, frames, T, D, H, cross=True, window_frames=window,
                                    map_frame_stride=stride)
            again = torch.empty_like(q)
            pl.layer_attention(q, k, v, again)
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"layer {layer}"
            assert torch.equal(again, out), f"layer {layer}"
    finally:
        pl.close()
