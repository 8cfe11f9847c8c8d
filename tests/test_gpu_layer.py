"""GPU parity of the whole-layer attention launch and of the split path's
edge cases, through the C-ABI.

* kvp_attn_forward_frames (every frame of a layer in one grid, frame f
  reading its own arena region and KVMap slice) against the CPU oracle,
  and bitwise equal to the same launch without a map.
* At C3's layer shape, where later workgroups walk their keys last to
  first, sampled rows of every frame match the oracle and a KVMap is
  bitwise invisible.
* Key rows past the end of a partial last tile never read the arena: an
  arena whose row 0 holds NaN leaves the output finite and bitwise equal to
  the map-free launch (T = 1560 is not a multiple of the 64-key tile).
* Split launches store fp16 partials scaled per query row: scaling V by 2^17
  (partials above fp16's 65504 without the row scale) or by 2^-20 (subnormal
  fp16 without it) scales the output by exactly that power of two, and the
  split output stays within the bf16 bar of the unsplit layer launch.
* Split launches on two streams at once give the results of serial runs.

Tolerances as in test_gpu_attention.py: fp32 max-abs <= 1e-3 / mean-abs
<= 1e-4, bf16 max-abs <= 2e-2 against the fp32 golden of bf16-rounded inputs.
"""

import numpy as np
import pytest
import torch

from kvpersist import api
from oracle import attention as at

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


def _dt(dtype):
    return api.FP32 if dtype == torch.float32 else api.BF16


def _check(got, want, dtype):
    err = (got - want).abs()
    if dtype == torch.float32:
        assert float(err.max()) <= FP32_MAX, float(err.max())
        assert float(err.mean()) <= FP32_MEAN, float(err.mean())
    else:
        assert float(err.max()) <= BF16_MAX, float(err.max())


def _layer_arenas(k, v, frames, T, mode, window, rng, region_rows):
    """Per-frame arena regions and KVMap slices: region f holds a random
    subset of frame f's key rows at permuted slots (slots < region_rows)."""
    D = k.shape[1]
    stride = frames * T if mode == "cross" else T
    arena = torch.zeros(frames * region_rows, 2 * D, dtype=k.dtype)
    kvmap = torch.full((frames * stride,), -1, dtype=torch.int64)
    for f in range(frames):
        b, e = at.key_range(mode, f, T, window)
        n = min(region_rows, e - b)
        rows = rng.choice(np.arange(b, e), size=n, replace=False)
        slots = rng.permutation(region_rows)[:n]
        for r, s in zip(rows, slots):
            arena[f * region_rows + s, :D] = k[r]
            arena[f * region_rows + s, D:] = v[r]
            kvmap[f * stride + (r if mode == "cross" else r - f * T)] = int(s)
    return arena, kvmap, stride


def _layer(dtype, qd, kd, vd, frames, T, heads, mode, window=0, arena=None, kvmap=None,
           region_bytes=0, map_stride=0):
    out = torch.empty_like(qd)
    api.attn_forward_frames(_dt(dtype), qd, kd, vd, arena, kvmap, out, frames, T,
                            heads * 128, heads, cross=(mode == "cross"), window_frames=window,
                            arena_frame_bytes=region_bytes, map_frame_stride=map_stride)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode,window", [("intra", 0), ("cross", 0), ("cross", 2)])
@pytest.mark.parametrize("T,heads", [(200, 2), (129, 3), (33, 1), (1560, 1)])
def test_layer_launch_matches_oracle_and_map_is_invisible(dtype, mode, window, T, heads):
    frames = 4
    q, k, v = _inputs(frames, T, heads, seed=T + 31 * heads, dtype=dtype)
    qd, kd, vd = (x.to(DEV).to(dtype).contiguous() for x in (q, k, v))
    base = _layer(dtype, qd, kd, vd, frames, T, heads, mode, window)
    want = at.attention_frames(q, k, v, frames, T, heads, mode, window)
    _check(base.float().cpu(), want, dtype)
    rng = np.random.default_rng(T)
    region_rows = max(1, T // 3)
    arena, kvmap, stride = _layer_arenas(k.to(dtype), v.to(dtype), frames, T, mode, window,
                                         rng, region_rows)
    region_bytes = region_rows * arena.shape[1] * arena.element_size()
    got = _layer(dtype, qd, kd, vd, frames, T, heads, mode, window, arena.to(DEV),
                 kvmap.to(DEV), region_bytes, stride)
    assert torch.equal(got, base)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("api_kind", ["single_frame", "layer"])
def test_kvmap_reads_the_arena_row_the_map_names(dtype, api_kind):
    """Arena rows hold other data than the key rows they stand in for: the
    output must be attention over K/V with every mapped row replaced by its
    arena row (reference semantics, src/gated_attention_kernel.cu:73-85 and
    :118-130), including rows in the last, partial key tile and two aligned
    16-row groups mapped to consecutive arena rows (the kernel's run path)."""
    frames, T, heads = 3, 1560, 2
    D = heads * 128
    q, k, v = _inputs(frames, T, heads, seed=29, dtype=dtype)
    rng = np.random.default_rng(29)
    region_rows = 200
    run_rows, run_slot0 = range(128, 160), region_rows  # slots past the permuted ones
    full = frames * T
    region_total = region_rows + len(run_rows)
    arena = torch.from_numpy(rng.standard_normal((frames * region_total, 2 * D),
                                                 dtype=np.float32))
    if dtype == torch.bfloat16:
        arena = at.round_bf16(arena)
    kvmap = torch.full((frames * full,), -1, dtype=torch.int64)
    want = torch.empty(frames * T, D)
    for f in range(frames):
        e = (f + 1) * T
        # whole 16-row groups, single rows, and rows of the last partial tile
        rows = set(rng.choice(e, size=120, replace=False).tolist())
        rows |= set(range(e - 20, e)) | set(range(64, 80))
        rows = sorted(rows - set(run_rows))[:region_rows]
        slots = list(rng.permutation(region_rows)[:len(rows)])
        rows += list(run_rows)
        slots += [run_slot0 + i for i in range(len(run_rows))]
        kf, vf = k[:e].clone(), v[:e].clone()
        for r, sl in zip(rows, slots):
            kvmap[f * full + r] = int(sl)
            kf[r] = arena[f * region_total + sl, :D]
            vf[r] = arena[f * region_total + sl, D:]
        want[f * T:e] = at.attention_keys(q[f * T:e], kf, vf, heads)
    qd, kd, vd = (x.to(DEV).to(dtype).contiguous() for x in (q, k, v))
    ad, md = arena.to(DEV).to(dtype), kvmap.to(DEV)
    if api_kind == "layer":
        got = _layer(dtype, qd, kd, vd, frames, T, heads, "cross", 0, ad, md,
                     region_total * 2 * D * ad.element_size(), full)
    else:
        got = torch.empty_like(qd)
        for f in range(frames):
            sl = slice(f * T, (f + 1) * T)
            fn = (api.attn_forward_single_frame if dtype == torch.float32
                  else api.attn_forward_single_frame_bf16)
            fn(qd[sl], kd, vd, ad[f * region_total:], md[f * full:(f + 1) * full], got[sl], T,
               D, heads, 1, f)
        torch.cuda.synchronize()
    _check(got.float().cpu(), want, dtype)


def test_cold_rows_nt_is_a_cache_hint_only():
    """Non-temporal loads of original rows change no output bit."""
    frames, T, heads = 4, 1560, 2
    q, k, v = _inputs(frames, T, heads, seed=61, dtype=torch.bfloat16)
    qd, kd, vd = (x.to(DEV).to(torch.bfloat16).contiguous() for x in (q, k, v))
    rng = np.random.default_rng(61)
    region_rows = 352
    arena, kvmap, stride = _layer_arenas(k.to(torch.bfloat16), v.to(torch.bfloat16), frames, T,
                                         "cross", 0, rng, region_rows)
    ad, md = arena.to(DEV), kvmap.to(DEV)
    outs = []
    for nt in (False, True):
        out = torch.empty_like(qd)
        api.attn_forward_frames(api.BF16, qd, kd, vd, ad, md, out, frames, T, heads * 128,
                                heads, cross=True, arena_frame_bytes=region_rows * 2 * 256 * 2,
                                map_frame_stride=stride, cold_rows_nt=nt)
        torch.cuda.synchronize()
        outs.append(out)
    assert torch.equal(outs[0], outs[1])
    assert torch.equal(outs[0], _layer(torch.bfloat16, qd, kd, vd, frames, T, heads, "cross"))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_layer_launch_equals_single_frame_launches_within_tolerance(dtype):
    # per-frame launches may split the key range; the layer launch never does
    frames, T, heads = 8, 1560, 2
    q, k, v = _inputs(frames, T, heads, seed=77, dtype=dtype)
    qd, kd, vd = (x.to(DEV).to(dtype).contiguous() for x in (q, k, v))
    layer = _layer(dtype, qd, kd, vd, frames, T, heads, "cross").float()
    per = torch.empty_like(qd)
    D = heads * 128
    for f in range(frames):
        sl = slice(f * T, (f + 1) * T)
        if dtype == torch.float32:
            api.attn_forward_single_frame(qd[sl], kd, vd, None, None, per[sl], T, D, heads, 1, f)
        else:
            api.attn_forward_single_frame_bf16(qd[sl], kd, vd, None, None, per[sl], T, D, heads,
                                               1, f)
    torch.cuda.synchronize()
    tol = 2e-5 if dtype == torch.float32 else 1.6e-2
    assert float((per.float() - layer).abs().max()) <= tol


@pytest.mark.parametrize("mode,window", [("cross", 0), ("cross", 3)])
def test_reversed_key_walks_match_oracle_and_map_is_invisible(mode, window):
    """C3's layer shape (8 x 1560, 12 heads: 1,248 workgroups, more than an
    MI355X XCD runs at once), so the workgroups that start after an XCD's
    first round walk their key tiles last to first: sampled query rows of
    every frame (first, middle and tail q-blocks) against the oracle; a KVMap
    with random arena rows is bitwise invisible; an arena whose row 0 holds
    NaN, with a sparse map that never names it, leaves the output finite and
    bitwise equal to the map-free launch."""
    frames, T, heads = 8, 1560, 12
    D = heads * 128
    q, k, v = _inputs(frames, T, heads, seed=1248 + window, dtype=torch.bfloat16)
    qd, kd, vd = (x.to(DEV).to(torch.bfloat16).contiguous() for x in (q, k, v))
    base = _layer(torch.bfloat16, qd, kd, vd, frames, T, heads, mode, window)
    got_all = base.float().cpu()
    for f in range(frames):
        b, e = at.key_range(mode, f, T, window)
        rows = np.r_[0:8, 700:708, T - 24:T] + f * T
        want = at.attention_keys(q[rows], k[b:e], v[b:e], heads)
        _check(got_all[rows], want, torch.bfloat16)
    rng = np.random.default_rng(99 + window)
    region_rows = 96
    arena, kvmap, stride = _layer_arenas(k.to(torch.bfloat16), v.to(torch.bfloat16), frames, T,
                                         mode, window, rng, region_rows)
    region_bytes = region_rows * 2 * D * 2
    got = _layer(torch.bfloat16, qd, kd, vd, frames, T, heads, mode, window, arena.to(DEV),
                 kvmap.to(DEV), region_bytes, stride)
    assert torch.equal(got, base)
    # slot 0 of every region unused by the map and poisoned
    kvmap = torch.where(kvmap == 0, torch.full_like(kvmap, -1), kvmap)
    for f in range(frames):
        arena[f * region_rows] = float("nan")
    got = _layer(torch.bfloat16, qd, kd, vd, frames, T, heads, mode, window, arena.to(DEV),
                 kvmap.to(DEV), region_bytes, stride)
    assert bool(torch.isfinite(got.float()).all())
    assert torch.equal(got, base)


@pytest.mark.parametrize("api_kind", ["single_frame", "layer"])
def test_rows_past_the_range_end_never_read_the_arena(api_kind):
    """Arena row 0 holds bf16 NaN; maps all -1, or sparse on rows >= 1 only."""
    frames, T, heads = 2, 1560, 2
    D = heads * 128
    q, k, v = _inputs(frames, T, heads, seed=5, dtype=torch.bfloat16)
    qd, kd, vd = (x.to(DEV).to(torch.bfloat16).contiguous() for x in (q, k, v))
    region_rows = 40
    arena = torch.zeros(frames * region_rows, 2 * D, dtype=torch.bfloat16)
    arena[0] = float("nan")
    arena[region_rows] = float("nan")
    full = frames * T
    maps = {"none": torch.full((frames * full,), -1, dtype=torch.int64)}
    sparse = maps["none"].clone()
    kb = k.to(torch.bfloat16)
    vb = v.to(torch.bfloat16)
    for f in range(frames):
        for s, r in enumerate(range(7, 7 + 3 * (region_rows - 1), 3)):
            if r < (f + 1) * T:
                arena[f * region_rows + s + 1, :D] = kb[r]
                arena[f * region_rows + s + 1, D:] = vb[r]
                sparse[f * full + r] = s + 1
    maps["sparse"] = sparse
    ad = arena.to(DEV)
    base = _layer(torch.bfloat16, qd, kd, vd, frames, T, heads, "cross")
    for name, m in maps.items():
        md = m.to(DEV)
        if api_kind == "layer":
            got = _layer(torch.bfloat16, qd, kd, vd, frames, T, heads, "cross", 0, ad, md,
                         region_rows * 2 * D * 2, full)
            ref = base
        else:
            got = torch.empty_like(qd)
            ref = torch.empty_like(qd)
            for f in range(frames):
                sl = slice(f * T, (f + 1) * T)
                api.attn_forward_single_frame_bf16(qd[sl], kd, vd, ad[f * region_rows:],
                                                   md[f * full:(f + 1) * full], got[sl], T, D,
                                                   heads, 1, f)
                api.attn_forward_single_frame_bf16(qd[sl], kd, vd, None, None, ref[sl], T, D,
                                                   heads, 1, f)
            torch.cuda.synchronize()
        assert bool(torch.isfinite(got.float()).all()), name
        assert torch.equal(got, ref), name


@pytest.mark.parametrize("exp2", [17, -20])
def test_split_partials_are_scale_invariant(exp2):
    frames, T, heads = 8, 1560, 2
    D = heads * 128
    f = frames - 1
    splits = api.attn_splits(api.BF16, T, heads, 1, frames * T)
    assert splits > 1, "this shape must take the split path"
    q, k, v = _inputs(frames, T, heads, seed=19, dtype=torch.bfloat16)
    qd, kd, vd = (x.to(DEV).to(torch.bfloat16).contiguous() for x in (q, k, v))
    scale = 2.0 ** exp2
    vs = (vd.float() * scale).to(torch.bfloat16)  # exact: a power of two
    assert torch.equal(vs.float(), vd.float() * scale)
    sl = slice(f * T, (f + 1) * T)
    outs = []
    for vv in (vd, vs):
        o = torch.empty(T, D, dtype=torch.bfloat16, device=DEV)
        api.attn_forward_single_frame_bf16(qd[sl], kd, vv, None, None, o, T, D, heads, 1, f)
        outs.append(o)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(outs[1].float()).all())
    assert torch.equal(outs[1].float(), outs[0].float() * scale)
    # against the unsplit layer launch and the oracle, relative to the scale
    layer = _layer(torch.bfloat16, qd, kd, vs, frames, T, heads, "cross")[sl].float()
    assert float((outs[1].float() - layer).abs().max()) <= BF16_MAX * scale
    rows = slice(0, 96)
    want = at.attention_keys(q[f * T:f * T + 96], k, v.float() * scale, heads)
    assert float((outs[1].float()[rows].cpu() - want).abs().max()) <= BF16_MAX * scale


def test_split_launches_on_two_streams_match_serial_runs():
    frames, T, heads = 8, 1560, 2
    D = heads * 128
    f = frames - 1
    assert api.attn_splits(api.BF16, T, heads, 1, frames * T) > 1
    ins = []
    for seed in (3, 4):
        q, k, v = _inputs(frames, T, heads, seed=seed, dtype=torch.bfloat16)
        ins.append(tuple(x.to(DEV).to(torch.bfloat16).contiguous() for x in (q, k, v)))
    sl = slice(f * T, (f + 1) * T)

    def launch(i, out, stream):
        qd, kd, vd = ins[i]
        api.attn_forward_range(api.BF16, qd[sl], kd, vd, None, None, out, T, D, heads, 0,
                               frames * T, stream)

    serial = []
    for i in range(2):
        o = torch.empty(T, D, dtype=torch.bfloat16, device=DEV)
        launch(i, o, torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        serial.append(o)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[torch.empty(T, D, dtype=torch.bfloat16, device=DEV) for _ in range(4)]
            for _ in range(2)]
    torch.cuda.synchronize()
    for rep in range(4):
        for i in range(2):
            launch(i, outs[i][rep], streams[i].cuda_stream)
    torch.cuda.synchronize()
    for i in range(2):
        for rep in range(4):
            assert torch.equal(outs[i][rep], serial[i]), (i, rep)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_softmax_keeps_o_finite_where_the_reference_does(dtype):
    """Unsplit layer launch (two frames, so no key split) on inputs where the
    scores jump by ~57 (log2 units) after the first tile and stay there, with
    V positive and ~2^64. The reference's online softmax keeps every weight
    <= 1 (src/gated_attention_kernel.cu:101-115), so its accumulator stays
    near keys x 2^64 ~ 2^73; an update that let a tile's weights sum to 2^63
    before rescaling would accumulate ~2^130 and overflow fp32. The output
    (the mean of the plateau keys' V rows) must be finite and match the
    float64 softmax within the precision bar, scaled by 2^64."""
    frames, T, heads = 2, 576, 1
    D = heads * 128
    scale = 2.0 ** 64
    q = torch.zeros(frames * T, D)
    q[:, 0] = 32.0
    k = torch.zeros(frames * T, D)
    for f in range(frames):
        k[f * T + 64:(f + 1) * T, 0] = 14.0  # q.k = 448: 57.1 in log2 units
    rng = np.random.default_rng(3)
    v = torch.from_numpy(rng.uniform(0.5, 1.5, (frames * T, D)).astype(np.float32)) * scale
    if dtype == torch.bfloat16:
        q, k, v = at.round_bf16(q), at.round_bf16(k), at.round_bf16(v)
    qd, kd, vd = (x.to(DEV).to(dtype).contiguous() for x in (q, k, v))
    got = _layer(dtype, qd, kd, vd, frames, T, heads, "intra").double().cpu()
    assert torch.isfinite(got).all()
    for f in range(frames):
        sl = slice(f * T, (f + 1) * T)
        s = (q[sl].double() @ k[sl].double().T) / np.sqrt(128.0)
        want = torch.softmax(s, dim=-1) @ v[sl].double()
        err = float((got[sl] - want).abs().max()) / scale
        assert err <= (FP32_MAX if dtype == torch.float32 else BF16_MAX), err


def test_split_workspaces_stay_bounded_across_streams():
    """Split launches on ten streams in turn: each stream's result equals the
    first, the library keeps at most 8 split workspaces on the device (least
    recently used freed), and releasing every stream's buffer leaves none of
    them behind."""
    from kvpersist import _lib
    lib = _lib.load()
    nq, keys, heads = 700, 4000, 4
    D = heads * 128
    g = torch.Generator(device=DEV).manual_seed(11)
    q, k, v = (torch.randn(n, D, generator=g, device=DEV).to(torch.bfloat16)
               for n in (nq, keys, keys))
    assert api.attn_splits(api.BF16, nq, heads, 1, keys) > 1
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(10)]
    outs = []
    for st in streams:
        o = torch.empty_like(q)
        assert lib.kvp_attn_forward_range(api.BF16, q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                          None, None, o.data_ptr(), nq, D, heads, 0, keys,
                                          st.cuda_stream) == 0
        st.synchronize()
        outs.append(o)
        assert lib.kvp_attn_workspace_count() <= 8
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    before = lib.kvp_attn_workspace_count()
    for st in streams:
        assert lib.kvp_attn_workspace_release(st.cuda_stream) == 0
    # the last 8 streams held buffers (the first two were evicted)
    assert lib.kvp_attn_workspace_count() == before - 8
