"""Product policies (C++ via the C-ABI) against the reference-built vectors.

tests/golden/policy_vectors.json holds the ids the reference's own
tile_gating_policy.cpp returns for 228 seeded score vectors (ties, zeros,
counts from 1 to 4900, budgets 0 to 300). The library must return exactly
those ids, and the window-aware select_range must agree with the oracle.
"""

import json
from pathlib import Path

import numpy as np
import pytest

from kvpersist import TileGatingPolicy
from oracle import policies as pol

CASES = json.loads((Path(__file__).parent / "golden" / "policy_vectors.json").read_text())["cases"]


def _scores(case):
    rng = np.random.default_rng(case["seed"])
    s = rng.random(case["n"], dtype=np.float32)
    if case.get("levels"):
        s = (np.floor(s * case["levels"]) / case["levels"]).astype(np.float32)
    if case.get("scale"):
        s = (s * np.float32(case["scale"])).astype(np.float32)
    return s


@pytest.mark.parametrize("policy", pol.POLICIES)
def test_library_policies_match_reference_vectors(policy):
    for case in CASES:
        p = TileGatingPolicy(policy, case["tpf"], case["total_frames"])
        got = p.select(_scores(case), case["n"], case["max"])
        assert got == case["expected"][policy], (policy, case["seed"])


@pytest.mark.parametrize("policy", pol.POLICIES)
def test_select_range_matches_oracle(policy):
    rng = np.random.default_rng(5)
    tpf, total = 98, 50
    for trial in range(40):
        frames_avail = int(rng.integers(1, 51))
        window = int(rng.integers(1, 9))
        first_frame = max(0, frames_avail - window)
        s = rng.random(frames_avail * tpf, dtype=np.float32)
        if trial % 4 == 0:
            s = np.round(s * 2).astype(np.float32)
        first = first_frame * tpf
        n = frames_avail * tpf - first
        m = int(rng.integers(0, 40))
        p = TileGatingPolicy(policy, tpf, total)
        got = p.select_range(s, first, n, m)
        want = pol.select_range(policy, s, first, n, m, tiles_per_frame=tpf, total_frames=total)
        assert got == want, (policy, trial)


def test_select_range_at_zero_equals_select():
    rng = np.random.default_rng(9)
    s = rng.random(784, dtype=np.float32)
    for policy in pol.POLICIES:
        p = TileGatingPolicy(policy, 98, 8)
        assert p.select_range(s, 0, 784, 22) == p.select(s, 784, 22)


def test_reuse_weighted_window_uses_absolute_source_frame():
    # candidates of frames 2..3 only (tpf 2): ids 4..7, total_frames 4
    s = np.zeros(8, dtype=np.float32)
    s[4:8] = [0.5, 0.0, 0.0, 0.5]
    p = TileGatingPolicy("reuse_weighted", 2, 4)
    # prio: id4 (4-2)*(1-1)=0, id5 2*1=2, id6 (4-3)*1=1, id7 0 -> [5, 6, 4, 7]
    assert p.select_range(s, 4, 4, 4) == [5, 6, 4, 7]
