"""Pins the CPU oracle before it is trusted as the checker.

Attention: float64 brute force, closed forms, and the reference's published
golden statistics of its own 8-frame seed-42 trace (regenerated bit-faithfully
by oracle.trace_synth). Policies: closed forms and vectors produced by the
reference's compiled policy code. Manager model: the reference capacity
scenario S1-S8 and hand-derived slot sequences. Planted-mistake cases show
that each pin rejects a plausible error.
"""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as at
from oracle import manager as mm
from oracle import policies as pol
from oracle import trace_synth as ts

GOLDEN = Path(__file__).parent / "golden"
META = json.loads((GOLDEN / "reference_meta.json").read_text())
VECTORS = json.loads((GOLDEN / "policy_vectors.json").read_text())["cases"]


def _rand(shape, seed):
    return torch.from_numpy(np.random.default_rng(seed).standard_normal(shape).astype(np.float32))


# ---------------------------------------------------------------- attention

@pytest.mark.parametrize("t,s,heads", [(37, 53, 2), (5, 1, 1), (64, 200, 3)])
def test_attention_matches_float64_bruteforce(t, s, heads):
    d = heads * 128
    q, k, v = _rand((t, d), 1), _rand((s, d), 2), _rand((s, d), 3)
    got = at.attention_keys(q, k, v, heads).numpy()
    want = at.attention_f64(q.numpy(), k.numpy(), v.numpy(), heads)
    assert np.abs(got - want).max() < 5e-6


def test_attention_single_key_returns_its_value_row():
    q, k, v = _rand((9, 256), 4), _rand((1, 256), 5), _rand((1, 256), 6)
    out = at.attention_keys(q, k, v, 2)
    assert torch.equal(out, v.expand(9, 256))


def test_attention_identical_keys_average_values():
    k = _rand((1, 128), 7).expand(40, 128).contiguous()
    v = _rand((40, 128), 8)
    out = at.attention_keys(_rand((3, 128), 9), k, v, 1)
    assert torch.allclose(out, v.mean(dim=0, keepdim=True).expand(3, 128), atol=1e-6)


def test_attention_rowsums_within_reference_tolerance():
    q, k, v = _rand((130, 256), 10), _rand((300, 256), 11), _rand((300, 256), 12)
    _, err = at.attention_keys(q, k, v, 2, return_rowsum_err=True)
    assert err < 1e-5  # reference: traces/gen_golden.py:116


def test_key_ranges():
    T = 1560
    assert at.key_range("intra", 3, T) == (3 * T, 4 * T)
    assert at.key_range("cross", 3, T) == (0, 4 * T)
    assert at.key_range("cross", 3, T, window_frames=8) == (0, 4 * T)
    assert at.key_range("cross", 9, T, window_frames=8) == (2 * T, 10 * T)
    assert at.key_range("cross", 7, T, window_frames=8) == (0, 8 * T)


@pytest.fixture(scope="module")
def trace8():
    torch.set_num_threads(max(1, min(8, torch.get_num_threads())))
    return ts.synthetic_trace(frames=8, seed=42)


def test_trace_regeneration_matches_reference_meta(trace8):
    ref = META["trace_8f"]
    static = trace8["static"]
    assert int(static.sum()) == ref["tiles"]["static"]
    assert int((~static).sum()) == ref["tiles"]["moving"]
    tok = torch.repeat_interleave(static, trace8["counts"])
    assert ts.cosine_report(trace8["k"], tok) == ref["validation_cosine_first_vs_last"]["K"]
    assert ts.cosine_report(trace8["v"], tok) == ref["validation_cosine_first_vs_last"]["V"]


def test_oracle_reproduces_reference_golden_statistics(trace8):
    """Per-frame mean/std (6 dp) of the reference's fp32 golden attention."""
    ref = META["golden_8f_intra"]
    worst = 0.0
    for st in ref["per_frame_stats"]:
        f = st["frame"]
        out, err = at.attention_keys(trace8["q"][f], trace8["k"][f], trace8["v"][f], 12,
                                     return_rowsum_err=True)
        worst = max(worst, err)
        assert round(float(out.mean()), 6) == st["mean"]
        assert round(float(out.std()), 6) == st["std"]
    assert worst < 1e-5


def test_planted_attention_mistakes_are_caught(trace8):
    """Each pin rejects a plausible mistake planted in a copy of the oracle."""
    q, k, v = trace8["q"][0], trace8["k"][0], trace8["v"][0]
    ref = META["golden_8f_intra"]["per_frame_stats"][0]
    # wrong scale (1/dh instead of 1/sqrt(dh)) -> golden std no longer matches
    wrong = at.attention_keys(q * (1.0 / math.sqrt(128.0)), k, v, 12)
    assert round(float(wrong.std()), 6) != ref["std"]
    # K and V swapped -> brute force disagrees
    qs, ks, vs = _rand((7, 128), 20), _rand((11, 128), 21), _rand((11, 128), 22)
    swapped = at.attention_keys(qs, vs, ks, 1).numpy()
    assert np.abs(swapped - at.attention_f64(qs.numpy(), ks.numpy(), vs.numpy(), 1)).max() > 1e-2
    # heads interleaved wrongly (dims as [dh, heads]) -> brute force disagrees
    q2, k2, v2 = _rand((6, 256), 23), _rand((9, 256), 24), _rand((9, 256), 25)
    perm = torch.arange(256).view(2, 128).t().reshape(-1)
    bad = at.attention_keys(q2[:, perm], k2[:, perm], v2[:, perm], 2)[:, perm.argsort()].numpy()
    assert np.abs(bad - at.attention_f64(q2.numpy(), k2.numpy(), v2.numpy(), 2)).max() > 1e-3


# ---------------------------------------------------------------- policies

def _scores(case):
    rng = np.random.default_rng(case["seed"])
    s = rng.random(case["n"], dtype=np.float32)
    if case.get("levels"):
        s = (np.floor(s * case["levels"]) / case["levels"]).astype(np.float32)
    if case.get("scale"):
        s = (s * np.float32(case["scale"])).astype(np.float32)
    assert float(s.astype(np.float64).sum()) == case["checksum"]
    return s


def test_policy_closed_forms():
    s = np.random.default_rng(0).random(50, dtype=np.float32)
    assert pol.select("none", s, 50, 10) == []
    assert pol.select("uniform", s, 50, 10) == list(range(10))
    assert pol.select("uniform", s, 3, 10) == list(range(10))  # ignores the count
    assert pol.select("recency", s, 50, 10) == list(range(40, 50))
    assert pol.select("recency", s, 4, 10) == [0, 1, 2, 3]
    assert pol.select("motion", s, 50, 10) == list(np.argsort(s, kind="stable")[:10])


def test_motion_ties_keep_id_order():
    s = np.array([0.5, 0.1, 0.5, 0.1, 0.3], dtype=np.float32)
    assert pol.select("motion", s, 5, 5) == [1, 3, 4, 0, 2]


def test_reuse_weighted_hand_case():
    # tpf 2, 3 frames: ids 0..5 from frames 0,0,1,1,2,2; rate_max 0.8
    s = np.array([0.4, 0.8, 0.0, 0.2, 0.4, 0.0], dtype=np.float32)
    # prio = remaining*(1-s/0.8): 3*.5, 0, 2*1, 2*.75, 1*.5, 1*1
    assert pol.select("reuse_weighted", s, 6, 6, tiles_per_frame=2, total_frames=3) == \
        [2, 0, 3, 5, 4, 1]


@pytest.mark.parametrize("policy", pol.POLICIES)
def test_oracle_policies_match_reference_vectors(policy):
    for case in VECTORS:
        s = _scores(case)
        got = pol.select(policy, s, case["n"], case["max"], tiles_per_frame=case["tpf"],
                         total_frames=case["total_frames"])
        assert got == case["expected"][policy], (policy, case["seed"])


def test_oracle_policies_against_live_reference_build():
    lib_path = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libref_policy.so"
    if not lib_path.exists():
        pytest.skip("oracle/_ref not built (needs /root/reference)")
    import ctypes
    lib = ctypes.CDLL(str(lib_path))
    lib.ref_policy_select.restype = ctypes.c_int
    lib.ref_policy_select.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.POINTER(ctypes.c_float), ctypes.c_int, ctypes.c_int,
                                      ctypes.POINTER(ctypes.c_long)]
    rng = np.random.default_rng(77)
    for trial in range(60):
        n = int(rng.integers(1, 3000))
        m = int(rng.integers(0, 120))
        tpf = int(rng.integers(1, 230))
        total = int(rng.integers(1, 60))
        s = rng.random(n, dtype=np.float32)
        if trial % 3 == 0:
            s = np.round(s * 3).astype(np.float32)
        buf = (ctypes.c_long * max(1, m))()
        for p in pol.POLICIES:
            k = lib.ref_policy_select(p.encode(), tpf, total,
                                      s.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n, m, buf)
            assert pol.select(p, s, n, m, tiles_per_frame=tpf, total_frames=total) == \
                [int(buf[i]) for i in range(k)], (p, trial)


def test_planted_policy_mistake_is_caught():
    case = next(c for c in VECTORS if c["n"] == 784 and c["max"] == 22 and c["levels"] == 4)
    s = _scores(case)
    # unstable sort would break ties differently
    unstable = list(np.argsort(-s, kind="quicksort")[::-1][:22])
    assert unstable != case["expected"]["motion"]


# ---------------------------------------------------------------- manager model

def test_manager_model_capacity_scenario_s1_s8():
    """reference: tests/test_capacity_admission.py:80-148."""
    g = META["grounding"]
    budget, tile, n = g["max_persisting_l2_bytes"], g["kv_tile_bytes"], g["tiles_fully_persistable"]
    assert budget // tile == n == 22
    m = mm.ManagerModel(budget, g["access_policy_max_window_bytes"])
    assert m.init() and m.query_device_limit() == budget                       # S1
    base = 0x10000
    adm = lambda i: m.admit(i, base + i * tile, tile)
    assert all(adm(i) == mm.ADMITTED for i in range(n))                        # S2
    assert m.used == budget and len(m.active) == n
    assert adm(n) == mm.REFUSED and m.used == budget                           # S3
    assert adm(5) == mm.INVALID and len(m.active) == n and m.used == budget    # S4
    assert m.release(7) and m.used == budget - tile and not m.release(7)       # S5
    assert adm(n) == mm.ADMITTED and len(m.active) == n                        # S6
    assert adm(n + 1) == mm.REFUSED
    m.clear()
    assert len(m.active) == 0 and m.used == 0 and adm(90) == mm.ADMITTED       # S7
    tpf, tt = g["tokens_per_frame"], g["tile_size_tokens"]                    # S8
    tiles = (tpf + tt - 1) // tt
    counts = [min(tt, tpf - i * tt) for i in range(tiles)]
    assert tiles == 98 and counts[-1] == 8 and sum(counts) == 1560


def test_manager_model_invalid_admits():
    m = mm.ManagerModel(1000, 500)
    assert m.admit(0, 1, 10) == mm.INVALID            # not initialised
    m.init()
    assert m.admit(-1, 1, 10) == mm.INVALID
    assert m.admit(0, 0, 10) == mm.INVALID
    assert m.admit(0, 1, 0) == mm.INVALID
    assert m.admit(0, 1, 501) == mm.INVALID           # above max window
    assert m.admit(0, 1, 500) == mm.ADMITTED
    assert m.admit(1, 1, 500) == mm.ADMITTED
    assert m.admit(2, 1, 1) == mm.REFUSED


def test_manager_model_arena_rows_sequential_and_refusal_keeps_state():
    m = mm.ManagerModel(3 * 100, 10 ** 9)
    m.init()
    assert m.arena_init(1000, 25)                     # stride 100 B
    assert not m.arena_init(1000, 25)                 # second init refused
    assert [m.arena_stage(50, 50) for _ in range(3)] == [0, 1, 2]
    assert m.arena_stage(50, 50) is None              # budget gate
    assert m.arena_used == 300 and m.next_row == 3
    m.arena_begin_step()
    assert m.arena_stage(50, 50) == 0


def test_manager_model_streaming_lifo_and_sticky():
    m = mm.ManagerModel(400, 10 ** 9)
    m.init()
    m.arena_init(400, 25)                             # 4 slots of 100 B
    assert m.streaming_begin()
    assert [m.streaming_stage(r, 50, 50)[1] for r in (10, 11, 12)] == [0, 1, 2]
    assert m.streaming_stage(11, 50, 50) == (True, 1, False)      # sticky hit
    assert m.streaming_stage(11, 50, 50, changed=True) == (True, 1, True)
    assert m.streaming_release(10) and m.streaming_release(12)
    assert not m.streaming_release(10)
    # LIFO: last released slot (2) comes back first, then 0, then the untouched 3
    assert [m.streaming_stage(r, 50, 50)[1] for r in (20, 21, 22)] == [2, 0, 3]
    assert m.streaming_stage(23, 50, 50) == (False, -1, False)    # capacity gate
    assert m.staged_bytes == 7 * 100 and m.high_water == 3


def test_plan_intra_streaming_release_quirk():
    """Intra + streaming releases rows of the current frame, so old slots never free
    (reference: src/run_policy_experiment.cu:180-185)."""
    T, tt, D = 64, 16, 128
    scores = np.array([[0.1, 0.2, 0.3, 0.4], [0.4, 0.3, 0.2, 0.1]], dtype=np.float32)
    # budget for exactly 2 fp32 tiles of 16 rows: 32 slots
    plan = mm.plan_frames("motion", cross=False, streaming=True, frames=2, T=T, D=D,
                          tile_tokens=tt, set_aside=2 * tt * D * 4 * 2, elem=4,
                          scores_flat=scores)
    assert plan[0]["ids"] == [0, 1] and plan[1]["ids"] == [3, 2]
    # frame 0 takes slots 0..31; frame 1 has no free slot left -> nothing staged
    assert sorted(s for _, s in plan[0]["copies"]) == list(range(32))
    assert plan[1]["copies"] == [] and plan[1]["staged_tiles"] == 0
    assert (plan[1]["map"][T:] == -1).all()
