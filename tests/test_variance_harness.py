"""Analysis of the fabric-read variance harness (kvpersist.variance) on
synthetic counter rows: launch window, ABBA order, spread gate, hot
launches, policy deltas and band separation (reference:
tests/test_variance.py:153-236)."""

import pytest

from kvpersist import variance as va


def _rows(n_attn, counter="FETCH_SIZE", other_every=3):
    rows, d = [], 0
    for i in range(n_attn):
        d += 1
        rows.append({"Dispatch_Id": str(d), "Kernel_Name": "void kvp::attn_fwd_bf16_kernel<x>",
                     "Counter_Name": counter, "Counter_Value": str(100.0 + i)})
        if i % other_every == 0:
            d += 1
            rows.append({"Dispatch_Id": str(d), "Kernel_Name": "attn_combine_kernel",
                         "Counter_Name": counter, "Counter_Value": "1e9"})
    rows.reverse()  # CSV order is not dispatch order
    return rows


def test_window_takes_launches_34_to_49_in_dispatch_order():
    got = va.window_bytes(_rows(50))
    assert got == [100.0 + i for i in range(34, 50)]


def test_window_sums_per_dispatch_and_ignores_other_counters():
    rows = _rows(50) + [dict(r, Counter_Name="TCC_HIT_sum") for r in _rows(50)]
    assert va.window_bytes(rows) == [100.0 + i for i in range(34, 50)]
    assert va.window_bytes(rows, counter="TCC_HIT_sum") == [100.0 + i for i in range(34, 50)]
    doubled = _rows(50) + _rows(50)  # two values under one dispatch id: summed
    assert va.window_bytes(doubled) == [2 * (100.0 + i) for i in range(34, 50)]


def test_window_counts_a_frames_combine_with_its_launch():
    # every third launch is followed by a combine dispatch (value 1e9)
    got = va.window_bytes(_rows(50), follow="attn_combine_kernel")
    assert got == [100.0 + i + (1e9 if i % 3 == 0 else 0.0) for i in range(34, 50)]
    f32 = [dict(r, Kernel_Name=r["Kernel_Name"].replace("bf16", "f32")) for r in _rows(50)]
    assert va.window_bytes(f32, kernel="attn_fwd_f32_kernel", follow="attn_combine_kernel") == got


def test_shapes_follow_the_reference_scoreboard():
    d = va.SHAPES["dense50"]
    assert d["dtype"] == "fp32" and d["window"] == 0 and d["set_aside"] == 2162688
    # 11 fp32 tiles of 16 rows x (K + V) x 1536 x 4 B (reference driver slot count)
    assert d["set_aside"] // (16 * 1536 * 4 * 2) == 11
    assert d["policies"] == ("none", "recency", "motion", "reuse_weighted")
    assert va.SHAPES["c4"]["window"] == 8


def test_window_needs_enough_launches():
    with pytest.raises(ValueError):
        va.window_bytes(_rows(49))


def test_abba_order():
    c = [("dense", "none"), ("dense", "motion"), ("stream", "none")]
    o = va.abba_orders(c, 3)
    assert o[0] == c and o[1] == list(reversed(c)) and o[2] == c


def test_spread_gate_and_median():
    s = va.combo_stats([100.0, 105.0, 110.0])
    assert s["median"] == 105.0 and s["min"] == 100.0 and s["max"] == 110.0
    assert abs(s["spread"] - 10.0 / 105.0) < 1e-12 and s["pass"]
    assert not va.combo_stats([100.0, 100.0, 112.0])["pass"]
    assert va.combo_stats([1.0, 3.0])["median"] == 2.0


def test_hot_launches_flag_ranges_above_20_percent():
    runs = [[10.0, 10.0, 10.0], [10.0, 13.0, 10.5], [10.0, 10.0, 10.0]]
    assert va.combo_stats([30.0, 33.5, 30.0], runs)["hot_launches"] == [1]


def test_policy_deltas_and_separation():
    mk = lambda lo, hi: {"median": 0.5 * (lo + hi), "min": lo, "max": hi}
    stats = {("dense", "none"): mk(100, 104), ("dense", "recency"): mk(90, 95),
             ("dense", "motion"): mk(101, 103), ("dense", "reuse_weighted"): mk(80, 85)}
    d = va.policy_deltas(stats, "dense")
    assert abs(d["recency"]["delta"] - (92.5 - 102) / 102) < 1e-12
    assert not d["recency"]["overlaps_none"] and d["motion"]["overlaps_none"]
    assert va.separated(stats, "dense")
    stats[("dense", "reuse_weighted")] = mk(94, 99)
    assert not va.separated(stats, "dense")
