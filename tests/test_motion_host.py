"""Host side of the motion producer mirror (kvpersist.motion) on the CPU:
the trace post-processing against the oracle, and the CSV round trip the
CLI and the variance harness read (reference:
traces/gen_motion_from_video.py:121-149, src/run_policy_experiment.cu:45-69)."""

import csv

import numpy as np

from kvpersist import motion
from oracle import farneback as fb


def test_trace_post_processing_matches_oracle():
    pairs = np.random.default_rng(2).random((7, 98)) * 9
    got = motion.trace_from_change(pairs, 40.0)
    want = fb.trace_from_change(pairs, 40.0)
    assert np.array_equal(got[0], want[0]) and got[1] == want[1]
    assert np.array_equal(got[2], want[2])


def test_csv_round_trip(tmp_path):
    pairs = np.random.default_rng(3).random((4, 98)) * 9
    change, tau, reuse = motion.trace_from_change(pairs)
    tr = motion.MotionTrace(change, tau, reuse, np.zeros((5, 30, 52)), 1560, 16, 50.0)
    p = tmp_path / "t.csv"
    with open(p, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["frame_id", "tile_id", "motion_score", "is_static", "token_start",
                    "token_count", "reuse"])
        w.writerows(motion.trace_rows(tr))
    assert [r[:6] for r in motion.trace_rows(tr)] == [r[:6] for r in fb.trace_rows(
        change, tau, reuse, 1560, 16)]
    s = motion.read_trace_csv(p)
    assert s.shape == (5, 98) and s.dtype == np.float32
    want = np.array([[np.float32(f"{v:.6f}") for v in row] for row in change])
    assert np.array_equal(s, want)
