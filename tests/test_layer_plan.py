"""Layer-mode planning of the frame pipeline (kvp_pipeline_run) against the
oracle driver model, on the CPU.

A plan-only pipeline makes every frame's plan a tile at a time (the batched
manager calls) and applies the staging launch's copy runs and map runs to
host copies of the layer map and of each physical row's source row; the
library refuses a launch whose runs would write one physical row or one map
entry twice. For every frame f of the layer:
  * slice f maps exactly the rows the oracle's frame-f map maps (reference
    driver loop: src/run_policy_experiment.cu:156-274), and nothing past the
    frame's key range;
  * each mapped row points at a physical row whose source is that row, rows
    of one frame at distinct physical rows;
a row keeps one physical row across the layer, physical rows are handed out
a tile at a time in key order, each tile the longest prefix of it any frame
maps (the copied rows are those prefixes, ascending; never more than
frames x rows-per-set-aside), and the last frame's introspection (selected
ids, staged tiles, rows copied, slot map, streaming bytes) equals the
oracle's. In bf16, each frame's group-descriptor table equals the table
kvp_attn_group_desc builds from that frame's map slice (two separate
encoders: the pipeline's from its tile segments, the builder's from the
entries). Layers are run back to back with different scores, so the map
runs and descriptor writes also cover entries that change or go back to -1
/ 0 between runs.
"""

import numpy as np
import pytest

from kvpersist import FramePipeline, api, workloads
from oracle import manager as mm

D = workloads.HIDDEN
HEADS = workloads.HEADS
TILE = 16


def _layer_pipeline(policy, *, cross, streaming, frames, T, set_aside, elem, window=0):
    return FramePipeline(policy, cross=cross, streaming=streaming, frames=frames, T=T, D=D,
                         heads=HEADS, tile_tokens=TILE, set_aside_bytes=set_aside,
                         dtype=0 if elem == 4 else 1, window_frames=window, plan_only=True)


def _check_layer(pl, policy, *, cross, streaming, frames, T, set_aside, elem, scores, window=0):
    plan = mm.plan_frames(policy, cross=cross, streaming=streaming, frames=frames, T=T, D=D,
                          tile_tokens=TILE, set_aside=set_aside, elem=elem, scores_flat=scores,
                          window_frames=window)
    pl.set_scores(scores)
    pl.run()
    last = plan[frames - 1]
    assert pl.selected() == last["ids"]
    if policy == "none":
        return
    assert pl.staged_tiles() == last["staged_tiles"]
    assert pl.copy_rows() == len(last["copies"])
    np.testing.assert_array_equal(pl.host_map()[:frames * T], last["map"])
    if streaming:
        assert pl.staged_bytes() == last["staged_bytes"]
    src = pl.layer_plan_sources()
    assert src.size == pl.layer_copied_rows()
    stride = frames * T if cross else T
    phys_of = {}
    prefix = {}  # tile -> longest mapped prefix over the frames
    tiles = (T + TILE - 1) // TILE
    for f in range(frames):
        sl = pl.layer_plan_map(f)
        assert sl.size == stride
        want = plan[f]["map"]  # slots over the frame's key rows [0, (f + 1) * T)
        if cross:
            got, rows0 = sl[:(f + 1) * T], 0
            assert (sl[(f + 1) * T:] == -1).all(), f
        else:
            want = want[f * T:(f + 1) * T]
            got, rows0 = sl, f * T
        np.testing.assert_array_equal(got >= 0, want >= 0, err_msg=f"{policy} frame {f}")
        rows = np.nonzero(got >= 0)[0]
        phys = got[rows]
        assert np.unique(phys).size == phys.size, f
        assert (phys < src.size).all(), f
        np.testing.assert_array_equal(src[phys], rows + rows0, err_msg=f"sources, frame {f}")
        for r, ph in zip((rows + rows0).tolist(), phys.tolist()):
            assert phys_of.setdefault(r, ph) == ph, (f, r)
        # each tile's mapped rows are a prefix of it
        per_tile = {}
        for r in (rows + rows0).tolist():
            g = r // T * tiles + (r % T) // TILE
            per_tile.setdefault(g, []).append(r - (r // T * T + (r % T) // TILE * TILE))
        for g, offs in per_tile.items():
            assert sorted(offs) == list(range(len(offs))), (f, g)
            prefix[g] = max(prefix.get(g, 0), len(offs))
        if elem == 2:
            b = max(0, f + 1 - window) * T if (cross and window) else 0
            e = (f + 1) * T if cross else T
            want_gd = api.attn_group_desc(sl, b, e, D)
            got_gd = pl.layer_plan_gd(f)
            n = want_gd.shape[0]
            assert got_gd.shape[0] >= n
            np.testing.assert_array_equal(got_gd[:n], want_gd, err_msg=f"descriptors, frame {f}")
            assert (got_gd[n:] == 0).all(), f
    # each touched tile's longest mapped prefix, once, in key order (so the
    # rows of adjacent fully mapped tiles sit in adjacent arena rows)
    want_src = [g // tiles * T + (g % tiles) * TILE + j for g in sorted(prefix)
                for j in range(prefix[g])]
    np.testing.assert_array_equal(src, want_src)
    assert src.size <= frames * (set_aside // (2 * D * elem))


CASES = [
    # name, cross, frames, T, window, set_aside (bytes), elem
    ("c3_22_tiles", True, 4, 1560, 0, workloads.CONFIGS["c3"].set_aside, 2),
    ("c3_88_tiles", True, 4, 1560, 0, 4 * workloads.CONFIGS["c3"].set_aside, 2),
    # 22 tiles and 9 spare rows (the slot count rounds down)
    ("c3_cut_tile", True, 4, 1560, 0, workloads.CONFIGS["c3"].set_aside + 9 * 2 * D * 2, 2),
    ("c4_window", True, 11, 1560, 8, workloads.CONFIGS["c4"].set_aside, 2),
    ("intra_fp32", False, 3, 1560, 0, workloads.CONFIGS["c2"].set_aside, 4),
    # T not a multiple of the tile: the last tile of a frame is short
    ("short_tail", True, 3, 1000, 0, 30 * TILE * D * 2 * 2 + 5 * 2 * D * 2, 2),
    # intra streaming keeps earlier frames' rows, so later frames run out of
    # slots part-way through a tile
    ("intra_cut", False, 3, 200, 0, 5 * TILE * D * 2 * 2 + 9 * 2 * D * 2, 2),
]


@pytest.mark.parametrize("policy", ["none", "uniform", "recency", "motion", "reuse_weighted"])
@pytest.mark.parametrize("streaming", [False, True])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_layer_plan_matches_oracle(case, streaming, policy):
    _, cross, frames, T, window, set_aside, elem = case
    tiles = (T + TILE - 1) // TILE
    rng = np.random.default_rng(frames * 1000 + T)
    pl = _layer_pipeline(policy, cross=cross, streaming=streaming, frames=frames, T=T,
                         set_aside=set_aside, elem=elem, window=window)
    try:
        # three layers back to back: scores A, B, A
        sa = rng.random((frames, tiles), dtype=np.float32)
        sb = rng.random((frames, tiles), dtype=np.float32)
        for sc in (sa, sb, sa):
            _check_layer(pl, policy, cross=cross, streaming=streaming, frames=frames, T=T,
                         set_aside=set_aside, elem=elem, scores=sc, window=window)
    finally:
        pl.close()


def test_layer_plan_motion_scores_c3_full():
    cfg = workloads.CONFIGS["c3"]
    scores = workloads.motion_for(cfg, 0)
    for streaming in (False, True):
        pl = _layer_pipeline("motion", cross=True, streaming=streaming, frames=cfg.frames,
                             T=cfg.tokens, set_aside=cfg.set_aside, elem=2)
        try:
            _check_layer(pl, "motion", cross=True, streaming=streaming, frames=cfg.frames,
                         T=cfg.tokens, set_aside=cfg.set_aside, elem=2, scores=scores)
        finally:
            pl.close()


@pytest.mark.parametrize("seed", [23, 30])
@pytest.mark.parametrize("policy", ["motion", "reuse_weighted"])
def test_layer_plan_partial_tile_shrinks_between_layers(seed, policy):
    """Scores (found by search) under which a frame maps fewer rows of a
    partly mapped tile than the previous layer did: the rows it no longer
    maps must go back to -1 in its map slice."""
    frames, T, tiles = 3, 200, 13
    set_aside = 5 * TILE * D * 2 * 2 + 9 * 2 * D * 2
    rng = np.random.default_rng(seed)
    pl = _layer_pipeline(policy, cross=False, streaming=True, frames=frames, T=T,
                         set_aside=set_aside, elem=2)
    try:
        for sc in [rng.random((frames, tiles), dtype=np.float32) for _ in range(3)]:
            _check_layer(pl, policy, cross=False, streaming=True, frames=frames, T=T,
                         set_aside=set_aside, elem=2, scores=sc)
    finally:
        pl.close()
