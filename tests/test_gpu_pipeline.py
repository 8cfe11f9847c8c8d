"""GPU parity of the full frame pipeline (select -> stage -> map -> attention).

Gates, as the reference harness has them (reference:
tests/test_policy_variants.py:174-179,228-230):
  * outputs bitwise equal across policies within a configuration;
  * streaming (sticky slots) outputs bitwise equal to dense arena outputs;
  * outputs within tolerance of the CPU golden.
Plus the invariants the arena must satisfy on the device:
  * the device KVMap equals the oracle driver's map, bit for bit;
  * every mapped row's arena slot holds exactly [K row | V row] (bitwise),
    i.e. the arena layout matches the reference manager's.
"""

import numpy as np
import pytest
import torch

from kvpersist import FramePipeline, workloads
from oracle import attention as at
from oracle import manager as mm

pytestmark = pytest.mark.gpu
DEV = "cuda"
D, HEADS = workloads.HIDDEN, workloads.HEADS


def _device_inputs(frames, T, dtype, seed):
    q, k, v = (torch.from_numpy(x) for x in workloads.qkv_host(frames, T, seed=seed))
    if dtype == torch.bfloat16:
        q, k, v = at.round_bf16(q), at.round_bf16(k), at.round_bf16(v)
    return q, k, v, q.to(DEV).to(dtype), k.to(DEV).to(dtype), v.to(DEV).to(dtype)


def _arena_rows(pl, nrows, dtype):
    n = nrows * 2 * D
    buf = torch.empty(n, dtype=dtype, device=DEV)
    esz = 4 if dtype == torch.float32 else 2
    torch.cuda.synchronize()
    from kvpersist import _lib
    lib = _lib.load()
    assert lib.kvp_memcpy_d2d(buf.data_ptr(), pl.arena_ptr(), n * esz, None) == 0
    torch.cuda.synchronize()
    return buf.view(nrows, 2 * D)


def _device_map(pl, n):
    from kvpersist import _lib
    lib = _lib.load()
    host = np.empty(n, dtype=np.int64)
    torch.cuda.synchronize()
    assert lib.kvp_memcpy_d2h(host.ctypes.data, pl.device_map_ptr(), n * 8, None) == 0
    return host


def _run_pipeline(policy, *, cross, streaming, frames, T, dtype, set_aside, scores, qkv,
                  window=0, check_arena=False):
    _, _, _, qd, kd, vd = qkv
    out = torch.empty_like(qd)
    d = 0 if dtype == torch.float32 else 1
    elem = 4 if dtype == torch.float32 else 2
    pl = FramePipeline(policy, cross=cross, streaming=streaming, frames=frames, T=T, D=D,
                       heads=HEADS, tile_tokens=16, set_aside_bytes=set_aside, dtype=d,
                       window_frames=window)
    pl.set_scores(scores)
    plan = None
    if check_arena and policy != "none":
        plan = mm.plan_frames(policy, cross=cross, streaming=streaming, frames=frames, T=T, D=D,
                              tile_tokens=16, set_aside=set_aside, elem=elem,
                              scores_flat=scores, window_frames=window)
    kflat, vflat = kd.view(frames * T, D), vd.view(frames * T, D)
    for f in range(frames):
        pl.step(f, qd, kd, vd, out)
        if plan is not None:
            dmap = _device_map(pl, (f + 1) * T)
            np.testing.assert_array_equal(dmap, plan[f]["map"], err_msg=f"map frame {f}")
            rows = np.nonzero(dmap >= 0)[0]
            if rows.size:
                cap = set_aside // (2 * D * elem)
                arena = _arena_rows(pl, cap, dtype)
                slots = torch.from_numpy(dmap[rows]).to(DEV)
                ridx = torch.from_numpy(rows).to(DEV)
                assert torch.equal(arena[slots, :D], kflat[ridx]), f
                assert torch.equal(arena[slots, D:], vflat[ridx]), f
    torch.cuda.synchronize()
    pl.close()
    return out


def test_c2_motion_arena_bit_exact_and_bitwise_output():
    cfg = workloads.CONFIGS["c2"]
    T = cfg.tokens
    qkv = _device_inputs(1, T, torch.float32, seed=42)
    scores = workloads.motion_for(cfg)
    base = _run_pipeline("none", cross=False, streaming=False, frames=1, T=T,
                         dtype=torch.float32, set_aside=0, scores=None, qkv=qkv)
    got = _run_pipeline("motion", cross=False, streaming=False, frames=1, T=T,
                        dtype=torch.float32, set_aside=cfg.set_aside, scores=scores, qkv=qkv,
                        check_arena=True)
    assert torch.equal(got, base)
    want = at.attention_keys(qkv[0], qkv[1], qkv[2], HEADS)
    err = (got.cpu() - want).abs()
    assert float(err.max()) <= 1e-3 and float(err.mean()) <= 1e-4


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cross_policies_bitwise_and_streaming_equals_dense(dtype):
    cfg = workloads.CONFIGS["c3"]
    frames, T = 4, cfg.tokens
    qkv = _device_inputs(frames, T, dtype, seed=5)
    scores = workloads.motion_for(cfg, 0)[:frames]
    set_aside = cfg.set_aside if dtype == torch.bfloat16 else 2 * cfg.set_aside
    base = _run_pipeline("none", cross=True, streaming=False, frames=frames, T=T, dtype=dtype,
                         set_aside=0, scores=None, qkv=qkv)
    for streaming in (False, True):
        for policy in ("uniform", "recency", "motion", "reuse_weighted"):
            got = _run_pipeline(policy, cross=True, streaming=streaming, frames=frames, T=T,
                                dtype=dtype, set_aside=set_aside, scores=scores, qkv=qkv,
                                check_arena=(policy == "motion"))
            assert torch.equal(got, base), (policy, streaming)
    # golden: frames 0 and 1 in full, the last frame on its first 256 queries
    q, k, v = qkv[0], qkv[1], qkv[2]
    tol = 1e-3 if dtype == torch.float32 else 2e-2
    outc = base.float().cpu()
    for f in (0, 1):
        want = at.attention_keys(q[f * T:(f + 1) * T], k[:(f + 1) * T], v[:(f + 1) * T], HEADS)
        assert float((outc[f * T:(f + 1) * T] - want).abs().max()) <= tol, f
    f = frames - 1
    want = at.attention_keys(q[f * T:f * T + 256], k[:(f + 1) * T], v[:(f + 1) * T], HEADS)
    assert float((outc[f * T:f * T + 256] - want).abs().max()) <= tol


def test_sliding_window_pipeline_bf16():
    cfg = workloads.CONFIGS["c4"]
    frames, T, W = 11, cfg.tokens, cfg.window
    qkv = _device_inputs(frames, T, torch.bfloat16, seed=8)
    scores = workloads.motion_for(cfg, 0)[:frames]
    base = _run_pipeline("none", cross=True, streaming=False, frames=frames, T=T,
                         dtype=torch.bfloat16, set_aside=0, scores=None, qkv=qkv, window=W)
    for policy in ("recency", "motion", "reuse_weighted"):
        got = _run_pipeline(policy, cross=True, streaming=True, frames=frames, T=T,
                            dtype=torch.bfloat16, set_aside=cfg.set_aside, scores=scores,
                            qkv=qkv, window=W, check_arena=(policy == "reuse_weighted"))
        assert torch.equal(got, base), policy
    q, k, v = qkv[0], qkv[1], qkv[2]
    f = frames - 1
    b = (f + 1 - W) * T
    want = at.attention_keys(q[f * T:f * T + 128], k[b:(f + 1) * T], v[b:(f + 1) * T], HEADS)
    assert float((base.float().cpu()[f * T:f * T + 128] - want).abs().max()) <= 2e-2


def test_c5_shape_single_frame_pair_bf16():
    cfg = workloads.CONFIGS["c5"]
    frames, T = 2, cfg.tokens
    qkv = _device_inputs(frames, T, torch.bfloat16, seed=9)
    scores = workloads.motion_for(cfg, 0)[:frames]
    base = _run_pipeline("none", cross=True, streaming=False, frames=frames, T=T,
                         dtype=torch.bfloat16, set_aside=0, scores=None, qkv=qkv)
    got = _run_pipeline("motion", cross=True, streaming=True, frames=frames, T=T,
                        dtype=torch.bfloat16, set_aside=cfg.set_aside, scores=scores, qkv=qkv,
                        check_arena=True)
    assert torch.equal(got, base)
    q, k, v = qkv[0], qkv[1], qkv[2]
    want = at.attention_keys(q[T:T + 128], k[:2 * T], v[:2 * T], HEADS)
    assert float((base.float().cpu()[T:T + 128] - want).abs().max()) <= 2e-2


def _layer_arena(pl, rows, dtype):
    n = rows * 2 * D
    buf = torch.empty(n, dtype=dtype, device=DEV)
    esz = 4 if dtype == torch.float32 else 2
    from kvpersist import _lib
    lib = _lib.load()
    torch.cuda.synchronize()
    assert lib.kvp_memcpy_d2d(buf.data_ptr(), pl.layer_arena_ptr(), n * esz, None) == 0
    torch.cuda.synchronize()
    return buf.view(rows, 2 * D)


def _layer_map(pl, f, n):
    from kvpersist import _lib
    lib = _lib.load()
    host = np.empty(n, dtype=np.int64)
    torch.cuda.synchronize()
    assert lib.kvp_memcpy_d2h(host.ctypes.data, pl.layer_map_ptr(f), n * 8, None) == 0
    return host


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("streaming", [False, True])
def test_run_layer_arena_and_maps_match_oracle_plan(dtype, streaming):
    """kvp_pipeline_run copies every row any frame of the layer maps into one
    layer arena, once, and writes frame f's KVMap to slice f of a layer map,
    then runs all frames in one launch. After the run, slice f must map
    exactly the rows the oracle driver's map of frame f maps, each to a
    distinct physical row holding [K row | V row]; a row keeps one physical
    row across frames; the copied rows are the union of the frames' mapped
    rows. Outputs are bitwise equal to policy none run the same way, and
    within the dtype's bar of frame-by-frame stepping (which may split key
    ranges)."""
    cfg = workloads.CONFIGS["c3"]
    frames, T = 4, cfg.tokens
    qkv = _device_inputs(frames, T, dtype, seed=9)
    _, _, _, qd, kd, vd = qkv
    scores = workloads.motion_for(cfg, 1)[:frames]
    set_aside = cfg.set_aside if dtype == torch.bfloat16 else 2 * cfg.set_aside
    elem = 4 if dtype == torch.float32 else 2
    d = 0 if dtype == torch.float32 else 1
    stepped = _run_pipeline("motion", cross=True, streaming=streaming, frames=frames, T=T,
                            dtype=dtype, set_aside=set_aside, scores=scores, qkv=qkv)
    outs = {}
    for policy in ("none", "motion"):
        pl = FramePipeline(policy, cross=True, streaming=streaming, frames=frames, T=T, D=D,
                           heads=HEADS, tile_tokens=16, set_aside_bytes=set_aside, dtype=d)
        pl.set_scores(scores)
        out = torch.empty_like(qd)
        for rep in range(2):  # a second pass reuses the pipeline's device state
            out.zero_()
            pl.run(qd, kd, vd, out)
            torch.cuda.synchronize()
            if rep == 0:
                first = out.clone()
            else:
                assert torch.equal(out, first)
        outs[policy] = out
        if policy == "motion":
            plan = mm.plan_frames("motion", cross=True, streaming=streaming, frames=frames, T=T,
                                  D=D, tile_tokens=16, set_aside=set_aside, elem=elem,
                                  scores_flat=scores)
            assert pl.layer_map_stride() == frames * T
            union = set()
            for f in range(frames):
                union.update(np.nonzero(plan[f]["map"] >= 0)[0].tolist())
            copied = pl.layer_copied_rows()
            assert copied == len(union)
            arena = _layer_arena(pl, copied, dtype)
            kflat, vflat = kd.view(frames * T, D), vd.view(frames * T, D)
            phys_of = {}
            for f in range(frames):
                dmap = _layer_map(pl, f, frames * T)
                want = plan[f]["map"]
                np.testing.assert_array_equal(dmap[:(f + 1) * T] >= 0, want >= 0,
                                              err_msg=f"mapped rows of slice {f}")
                assert (dmap[(f + 1) * T:] == -1).all(), f
                rows = np.nonzero(dmap >= 0)[0]
                assert rows.size > 0
                phys = dmap[rows]
                assert phys.max() < copied and np.unique(phys).size == phys.size, f
                for r, ph in zip(rows.tolist(), phys.tolist()):
                    assert phys_of.setdefault(r, ph) == ph, (f, r)
                pidx = torch.from_numpy(phys).to(DEV)
                ridx = torch.from_numpy(rows).to(DEV)
                assert torch.equal(arena[pidx, :D], kflat[ridx]), f
                assert torch.equal(arena[pidx, D:], vflat[ridx]), f
        pl.close()
    assert torch.equal(outs["motion"], outs["none"])
    tol = 2e-5 if dtype == torch.float32 else 1.6e-2
    assert float((outs["motion"].float() - stepped.float()).abs().max()) <= tol


def test_failed_layer_run_leaves_the_next_run_correct():
    """A layer run whose staging launch is refused (K and V 2 bytes off
    16-byte alignment: refused on the host, nothing reaches the device)
    fails after the pipeline's host mirrors of the device map and descriptor
    tables were updated for it. The next run must still leave every map
    slice and descriptor table exactly as a plan-only pipeline plans them
    for that run's scores, and give policy none's output bit for bit."""
    from kvpersist import _lib, api
    lib = _lib.load()
    cfg = workloads.CONFIGS["c3"]
    frames, T = 3, cfg.tokens
    _, _, _, qd, kd, vd = _device_inputs(frames, T, torch.bfloat16, seed=17)
    rng = np.random.default_rng(17)
    tiles = (T + 15) // 16
    sa, sb, sc = (rng.random((frames, tiles), dtype=np.float32) for _ in range(3))
    kw = dict(cross=True, streaming=False, frames=frames, T=T, D=D, heads=HEADS,
              tile_tokens=16, set_aside_bytes=cfg.set_aside, dtype=api.BF16)
    pl = FramePipeline("motion", **kw)
    out = torch.empty_like(qd)
    pl.set_scores(sa)
    pl.run(qd, kd, vd, out)
    torch.cuda.synchronize()
    # the same K/V bytes, 2 bytes off alignment
    kbuf = torch.empty(kd.numel() + 8, dtype=torch.bfloat16, device=DEV)
    vbuf = torch.empty_like(kbuf)
    kbuf[1:1 + kd.numel()] = kd.view(-1)
    vbuf[1:1 + vd.numel()] = vd.view(-1)
    pl.set_scores(sb)
    with pytest.raises(RuntimeError):
        pl.run(qd, kbuf[1:1 + kd.numel()].view_as(kd), vbuf[1:1 + vd.numel()].view_as(vd), out)
    pl.set_scores(sc)
    pl.run(qd, kd, vd, out)
    torch.cuda.synchronize()
    plan = FramePipeline("motion", plan_only=True, **kw)
    plan.set_scores(sc)
    plan.run()
    stride, gstride = pl.layer_map_stride(), pl.layer_gd_stride()
    for f in range(frames):
        np.testing.assert_array_equal(_layer_map(pl, f, stride), plan.layer_plan_map(f),
                                      err_msg=f"slice {f}")
        gd = np.empty((gstride, 2), dtype=np.uint32)
        assert lib.kvp_memcpy_d2h(gd.ctypes.data, pl.layer_gd_ptr() + 8 * f * gstride,
                                  gd.nbytes, None) == 0
        np.testing.assert_array_equal(gd, plan.layer_plan_gd(f), err_msg=f"descriptors {f}")
    nb = FramePipeline("none", **kw)
    ref = torch.empty_like(qd)
    nb.run(qd, kd, vd, ref)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    for p in (pl, plan, nb):
        p.close()
