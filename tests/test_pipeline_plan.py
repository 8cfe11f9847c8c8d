"""Host bookkeeping of the frame pipeline against the oracle driver model.

The C++ pipeline runs in plan-only mode (no device work): for every frame
the selected ids, the KVMap prefix, the number of staged tiles and the rows
copied must equal the oracle's restatement of the reference driver loop
(reference: src/run_policy_experiment.cu:156-274), bit for bit. Covers all
five policies, intra / cross / sliding window, dense arena and streaming
slots, fp32 and bf16 row sizes, at the benchmark configurations' shapes.
"""

import numpy as np
import pytest

from kvpersist import FramePipeline, workloads
from oracle import manager as mm

D = workloads.HIDDEN
HEADS = workloads.HEADS


def _compare(policy, *, cross, streaming, frames, T, set_aside, elem, scores, window=0):
    dtype = 0 if elem == 4 else 1
    pl = FramePipeline(policy, cross=cross, streaming=streaming, frames=frames, T=T, D=D,
                       heads=HEADS, tile_tokens=16, set_aside_bytes=set_aside, dtype=dtype,
                       window_frames=window, plan_only=True)
    pl.set_scores(scores)
    plan = mm.plan_frames(policy, cross=cross, streaming=streaming, frames=frames, T=T, D=D,
                          tile_tokens=16, set_aside=set_aside, elem=elem, scores_flat=scores,
                          window_frames=window)
    for f in range(frames):
        pl.step(f)
        exp = plan[f]
        assert pl.selected() == exp["ids"], (policy, f)
        if policy == "none":
            continue
        assert pl.staged_tiles() == exp["staged_tiles"], (policy, f)
        assert pl.copy_rows() == len(exp["copies"]), (policy, f)
        got_map = pl.host_map()[:(f + 1) * T]
        np.testing.assert_array_equal(got_map, exp["map"], err_msg=f"{policy} frame {f}")
        if streaming and f == frames - 1:
            assert pl.staged_bytes() == exp["staged_bytes"]
    pl.close()
    return plan


def test_c2_motion_arena_plan():
    cfg = workloads.CONFIGS["c2"]
    scores = workloads.motion_for(cfg)
    plan = _compare("motion", cross=False, streaming=False, frames=1, T=cfg.tokens,
                    set_aside=cfg.set_aside, elem=4, scores=scores)
    # 22 tiles admitted; arena rows are handed out 0, 1, 2, ... in staging order
    ids = plan[0]["ids"]
    rows = sum(min(16, cfg.tokens - 16 * t) for t in ids)
    assert len(ids) == 22 and plan[0]["staged_tiles"] == 22
    assert [s for _, s in plan[0]["copies"]] == list(range(rows))
    assert [r for r, _ in plan[0]["copies"]] == [16 * t + i for t in ids
                                                 for i in range(min(16, cfg.tokens - 16 * t))]


@pytest.mark.parametrize("policy", ["none", "uniform", "recency", "motion", "reuse_weighted"])
@pytest.mark.parametrize("streaming", [False, True])
def test_c3_cross_plan(policy, streaming):
    cfg = workloads.CONFIGS["c3"]
    _compare(policy, cross=True, streaming=streaming, frames=cfg.frames, T=cfg.tokens,
             set_aside=cfg.set_aside, elem=2, scores=workloads.motion_for(cfg, 0))


@pytest.mark.parametrize("policy", ["uniform", "motion"])
@pytest.mark.parametrize("streaming", [False, True])
def test_intra_plan(policy, streaming):
    cfg = workloads.CONFIGS["c3"]
    _compare(policy, cross=False, streaming=streaming, frames=4, T=cfg.tokens,
             set_aside=4 * workloads.FP32_TILE_BYTES, elem=4,
             scores=workloads.motion_for(cfg, 1)[:4])


@pytest.mark.parametrize("policy", ["recency", "motion", "reuse_weighted"])
@pytest.mark.parametrize("streaming", [False, True])
def test_c4_window_plan(policy, streaming):
    cfg = workloads.CONFIGS["c4"]
    frames = 14  # crosses the 8-frame window boundary
    _compare(policy, cross=True, streaming=streaming, frames=frames, T=cfg.tokens,
             set_aside=cfg.set_aside, elem=2,
             scores=workloads.motion_for(cfg, 0)[:frames], window=cfg.window)


def test_c5_plan():
    cfg = workloads.CONFIGS["c5"]
    _compare("motion", cross=True, streaming=True, frames=6, T=cfg.tokens,
             set_aside=cfg.set_aside, elem=2, scores=workloads.motion_for(cfg, 0)[:6])


def test_partial_tile_and_small_budget():
    # 100 tokens -> 7 tiles, last holds 4 rows; budget of 3 fp32 tiles.
    T = 100
    rng = np.random.default_rng(3)
    scores = rng.random((5, 7), dtype=np.float32)
    scores[:, 6] = 0.0  # force the short tile into the motion selection
    for streaming in (False, True):
        _compare("motion", cross=True, streaming=streaming, frames=5, T=T,
                 set_aside=3 * 16 * D * 4 * 2, elem=4, scores=scores)
        _compare("motion", cross=False, streaming=streaming, frames=5, T=T,
                 set_aside=3 * 16 * D * 4 * 2, elem=4, scores=scores)


def test_uniform_budget_above_tile_count():
    # uniform ignores the candidate count: ids beyond the frame's tiles stage nothing
    T = 48  # 3 tiles
    scores = np.zeros((2, 3), dtype=np.float32)
    _compare("uniform", cross=False, streaming=False, frames=2, T=T,
             set_aside=5 * 16 * D * 4 * 2, elem=4, scores=scores)
