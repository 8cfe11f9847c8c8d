"""Hand-derived pins of the cross-frame driver plan.

Each case below was worked out by hand from the reference driver loop
(reference: src/run_policy_experiment.cu:156-232) and the streaming slot
rules (reference: src/kv_tile_manager.cu:141-200), not by running any code:

* a selected candidate gid of frame f's prefix is source frame gid // 3,
  tile gid % 3; its rows are src_f * T + 16 * tile + r (cross mode keys the
  map by absolute row);
* streaming: the tiles that dropped out of the selection are released
  before anything is staged, walking gid ascending and rows ascending, and
  each release pushes the row's slot onto the back of the free list;
* staging pops slots from the back of the free list (slot 0 first after
  streaming_begin), so a tile admitted right after two released tiles gets
  their slots in reverse;
* arena mode hands out rows 0, 1, 2, ... in staging order, every frame.

Geometry: T = 48 tokens (3 tiles of 16; T = 40 for the short-tile case),
one head (D = 128), fp32 rows, budget = 2 tiles = 32 rows of arena.

The oracle's plan_frames and the library pipeline (plan-only mode) must
reproduce every expected map and copy list. The planted mistakes — the
source row without its frame term, the release after staging, the release
walking dropped tiles in descending order — must each break at least one
case.
"""

import numpy as np
import pytest

from kvpersist import FramePipeline
from oracle import manager as mm

D, TT = 128, 16
BUDGET = 2 * TT * D * 4 * 2  # two fp32 tiles = 32 arena rows

# scores[frame][tile], frame-major
MOTION = np.array([[0.5, 0.1, 0.9],
                   [0.2, 0.8, 0.7],
                   [0.05, 0.6, 0.3]], dtype=np.float32)


def _rows(r0, r1, s0, s1):
    """Rows r0..r1 (inclusive) mapped to slots s0..s1, stepping up or down."""
    step = 1 if s1 >= s0 else -1
    slots = list(range(s0, s1 + step, step))
    rows = list(range(r0, r1 + 1))
    assert len(rows) == len(slots)
    return list(zip(rows, slots))


def _map(n, *runs):
    m = np.full(n, -1, dtype=np.int64)
    for run in runs:
        for r, s in run:
            m[r] = s
    return m


# name -> (policy, streaming, T, frames, window, scores, per-frame expected)
# expected per frame: (ids, map prefix, copies)
CASES = {
    # recency keeps the newest two tiles; every frame drops both and stages
    # two new ones, so the LIFO list alternates between handing slots out
    # ascending and descending.
    "recency_stream": ("recency", True, 48, 4, 0, np.zeros((4, 3), np.float32), [
        ([1, 2], _map(48, _rows(16, 31, 0, 15), _rows(32, 47, 16, 31)),
         _rows(16, 31, 0, 15) + _rows(32, 47, 16, 31)),
        # release gid 1 (rows 16..31 -> push 0..15), gid 2 (push 16..31):
        # free list back is 31
        ([4, 5], _map(96, _rows(64, 79, 31, 16), _rows(80, 95, 15, 0)),
         _rows(64, 79, 31, 16) + _rows(80, 95, 15, 0)),
        # release gid 4 (rows 64..79 -> push 31..16), gid 5 (push 15..0)
        ([7, 8], _map(144, _rows(112, 127, 0, 15), _rows(128, 143, 16, 31)),
         _rows(112, 127, 0, 15) + _rows(128, 143, 16, 31)),
        ([10, 11], _map(192, _rows(160, 175, 31, 16), _rows(176, 191, 15, 0)),
         _rows(160, 175, 31, 16) + _rows(176, 191, 15, 0)),
    ]),
    # motion picks the two lowest scores of the prefix; tile gid 1 stays
    # selected for three frames (sticky: no copy, same slots).
    "motion_stream": ("motion", True, 48, 3, 0, MOTION, [
        ([1, 0], _map(48, _rows(16, 31, 0, 15), _rows(0, 15, 16, 31)),
         _rows(16, 31, 0, 15) + _rows(0, 15, 16, 31)),
        # prefix order: gid1 .1, gid3 .2, gid0 .5 -> [1, 3]; gid 0 released
        # (push 16..31); gid 3 = frame 1 tile 0 = rows 48..63 pops 31..16
        ([1, 3], _map(96, _rows(16, 31, 0, 15), _rows(48, 63, 31, 16)),
         _rows(48, 63, 31, 16)),
        # prefix order: gid6 .05, gid1 .1 -> [6, 1]; gid 3 released (rows
        # 48..63 push 31..16, back 16); gid 6 = rows 96..111 pops 16..31
        ([6, 1], _map(144, _rows(96, 111, 16, 31), _rows(16, 31, 0, 15)),
         _rows(96, 111, 16, 31)),
    ]),
    # arena mode: rows restart at 0 every frame, in staging order
    "motion_arena": ("motion", False, 48, 3, 0, MOTION, [
        ([1, 0], _map(48, _rows(16, 31, 0, 15), _rows(0, 15, 16, 31)),
         _rows(16, 31, 0, 15) + _rows(0, 15, 16, 31)),
        ([1, 3], _map(96, _rows(16, 31, 0, 15), _rows(48, 63, 16, 31)),
         _rows(16, 31, 0, 15) + _rows(48, 63, 16, 31)),
        ([6, 1], _map(144, _rows(96, 111, 0, 15), _rows(16, 31, 16, 31)),
         _rows(96, 111, 0, 15) + _rows(16, 31, 16, 31)),
    ]),
    # window of 2 frames: frame 2 sees candidates gid 3..8 only -> [6, 3];
    # gid 1 is released (rows 16..31 push 0..15, back 15), gid 6 pops 15..0,
    # gid 3 keeps its slots
    "motion_stream_window2": ("motion", True, 48, 3, 2, MOTION, [
        ([1, 0], _map(48, _rows(16, 31, 0, 15), _rows(0, 15, 16, 31)),
         _rows(16, 31, 0, 15) + _rows(0, 15, 16, 31)),
        ([1, 3], _map(96, _rows(16, 31, 0, 15), _rows(48, 63, 31, 16)),
         _rows(48, 63, 31, 16)),
        ([6, 3], _map(144, _rows(96, 111, 15, 0), _rows(48, 63, 31, 16)),
         _rows(96, 111, 15, 0)),
    ]),
    # T = 40: tiles of 16, 16 and 8 rows; frame 1 starts at row 40
    "recency_arena_short_tile": ("recency", False, 40, 2, 0, np.zeros((2, 3), np.float32), [
        ([1, 2], _map(40, _rows(16, 31, 0, 15), _rows(32, 39, 16, 23)),
         _rows(16, 31, 0, 15) + _rows(32, 39, 16, 23)),
        ([4, 5], _map(80, _rows(56, 71, 0, 15), _rows(72, 79, 16, 23)),
         _rows(56, 71, 0, 15) + _rows(72, 79, 16, 23)),
    ]),
}


def _oracle(name, plant=None):
    policy, streaming, T, frames, window, scores, _ = CASES[name]
    return mm.plan_frames(policy, cross=True, streaming=streaming, frames=frames, T=T, D=D,
                          tile_tokens=TT, set_aside=BUDGET, elem=4, scores_flat=scores,
                          window_frames=window, _plant=plant)


def _matches(plan, expected):
    for got, (ids, m, copies) in zip(plan, expected):
        if got["ids"] != ids or list(got["copies"]) != copies:
            return False
        if not np.array_equal(got["map"], m):
            return False
    return True


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_plan_matches_hand_derivation(name):
    expected = CASES[name][-1]
    plan = _oracle(name)
    assert len(plan) == len(expected)
    for f, (got, (ids, m, copies)) in enumerate(zip(plan, expected)):
        assert got["ids"] == ids, (name, f)
        np.testing.assert_array_equal(got["map"], m, err_msg=f"{name} frame {f}")
        assert list(got["copies"]) == copies, (name, f)
        assert got["staged_tiles"] == len(ids), (name, f)


@pytest.mark.parametrize("name", sorted(CASES))
def test_library_plan_matches_hand_derivation(name):
    policy, streaming, T, frames, window, scores, expected = CASES[name]
    pl = FramePipeline(policy, cross=True, streaming=streaming, frames=frames, T=T, D=D,
                       heads=1, tile_tokens=TT, set_aside_bytes=BUDGET, dtype=0,
                       window_frames=window, plan_only=True)
    pl.set_scores(scores)
    try:
        for f, (ids, m, copies) in enumerate(expected):
            pl.step(f)
            assert pl.selected() == ids, (name, f)
            np.testing.assert_array_equal(pl.host_map()[:(f + 1) * T], m,
                                          err_msg=f"{name} frame {f}")
            assert pl.copy_rows() == len(copies), (name, f)
            assert pl.staged_tiles() == len(ids), (name, f)
    finally:
        pl.close()


@pytest.mark.parametrize("plant", mm.PLANTS)
def test_planted_plan_mistakes_are_caught(plant):
    caught = [name for name in CASES if not _matches(_oracle(name, plant), CASES[name][-1])]
    assert caught, f"planted mistake {plant} passes every hand-derived case"


def test_each_planted_mistake_breaks_the_recency_stream_case():
    # the case that exercises all three: frame-offset rows, release before
    # staging (capacity is full after frame 0) and ascending release order
    # (the reversed slot hand-out of frame 1)
    for plant in mm.PLANTS:
        assert not _matches(_oracle("recency_stream", plant), CASES["recency_stream"][-1]), plant
