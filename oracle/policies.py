"""Tile gating policies, numpy restatement. TEST INFRASTRUCTURE ONLY.

Rules (reference: src/tile_gating_policy.cpp):
  none            []                                              (:6-11)
  uniform         [0, max)                                        (:13-19)
  recency         [max(0, n - max), n)                            (:21-30)
  reuse_weighted  rate_max = max(1e-6f, max s) in float32,
                  prio = (total_frames - id // tpf) * (1 - min(1, s / rate_max))
                  in float64, order by prio desc then id asc, take max  (:32-68)
  motion          stable ascending sort of float32 scores, take max  (:70-83)

select_range(first, n) applies the rule to candidates first..first+n-1 and
returns absolute ids; reuse_weighted takes the source frame of an absolute
id (the window-aware form of the library).

Pinned by (tests/test_oracle_pins.py): closed forms for none / uniform /
recency; numpy.argsort(kind="stable") equivalence and hand-checked
tie cases for motion; for every policy, vectors produced by compiling the
reference's own tile_gating_policy.cpp into oracle/_ref (committed as
tests/golden/policy_vectors.json, and re-checked live when oracle/_ref is
built).
"""

from __future__ import annotations

import numpy as np

POLICIES = ("none", "uniform", "recency", "motion", "reuse_weighted")


def select(name: str, scores, num_candidates: int, max_tiles: int, *,
           tiles_per_frame: int = 1, total_frames: int = 1) -> list[int]:
    return select_range(name, scores, 0, num_candidates, max_tiles,
                        tiles_per_frame=tiles_per_frame, total_frames=total_frames)


def select_range(name: str, scores_flat, first_id: int, num_candidates: int, max_tiles: int, *,
                 tiles_per_frame: int = 1, total_frames: int = 1) -> list[int]:
    n = max(0, int(num_candidates))
    m = max(0, int(max_tiles))
    if name == "none":
        return []
    if name == "uniform":
        return [first_id + i for i in range(m)]
    if name == "recency":
        return [first_id + i for i in range(max(0, n - m), n)]
    s = np.asarray(scores_flat, dtype=np.float32)[first_id:first_id + n]
    if name == "motion":
        order = np.argsort(s, kind="stable")
        return [first_id + int(i) for i in order[:min(m, n)]]
    if name == "reuse_weighted":
        rate_max = np.float32(1e-6)
        if n:
            rate_max = max(rate_max, np.float32(s.max()))
        ids = np.arange(first_id, first_id + n, dtype=np.int64)
        remaining = (total_frames - ids // max(1, tiles_per_frame)).astype(np.float64)
        rate = np.minimum(1.0, s.astype(np.float64) / np.float64(rate_max))
        prio = remaining * (1.0 - rate)
        order = np.lexsort((ids, -prio))  # prio descending, ties by id
        return [int(ids[i]) for i in order[:min(m, n)]]
    raise ValueError(f"unknown policy {name!r}")
