"""Group-descriptor tables of a KVMap slice (kvp_attn_group_desc; format in
kvp_c_api.h next to kvp_attn_forward_frames_gd), on the CPU.

The bf16 attention kernel reads one descriptor entry per 16-row copy group
instead of the group's 16 map entries, so a table must say, for every key
row, exactly what the map says: the arena row the entry names when the bf16
kernel honours it (0 <= m and 2 (m + 1) 2D <= 2^32), else "original row"
(reference map semantics: src/gated_attention_kernel.cu:73-85, :118-130).
Checked by decoding each entry with a decoder written from the documented
bit layout (not from the encoder), on hand-built groups whose words are
derived by hand, and on random maps with runs, reversed runs, holes, single
entries, entries past the 32-bit reach and negative values other than -1,
over ranges that start off the 16-row grid. A "general" entry must be used
only for a group whose arena rows form more than two runs.
"""

import numpy as np
import pytest

from kvpersist import api

D = 1536
MAX_ROW = 2**31 // (2 * D) - 1  # 2 (m + 1) 2D <= 2^32


def honoured(m):
    return m if 0 <= m <= MAX_ROW else -1


def decode(gd, b, e):
    """Arena row per key row of [b, e) (-1: original row) and a mask of rows
    in general groups, from the documented layout."""
    n = e - b
    rows = np.full(n, -1, dtype=np.int64)
    general = np.zeros(n, dtype=bool)
    assert gd.shape == (4 * ((n + 63) // 64), 2)
    for g in range(gd.shape[0]):
        w0, w1 = int(gd[g, 0]), int(gd[g, 1])
        lo, hi = 16 * g, min(16 * g + 16, n)
        if w0 == 0:
            assert w1 == 0
            continue
        if w0 == 1:
            assert w1 == 0 and lo < n
            general[lo:hi] = True
            continue
        for w in (w0, w1):
            if w == 0:
                continue
            assert w >> 31 == 1
            l, r0, cnt = w & 0x7FFFFF, (w >> 23) & 15, ((w >> 27) & 15) + 1
            assert r0 + cnt <= 16 and lo + r0 + cnt <= hi, (g, hex(w))
            for i in range(cnt):
                assert rows[lo + r0 + i] == -1, "sub-runs overlap"
                rows[lo + r0 + i] = l + i
    return rows, general


def runs_in(vals):
    """Number of maximal runs of consecutive rows with consecutive arena rows."""
    runs, prev = 0, None
    for m in vals:
        if m >= 0 and (prev is None or prev < 0 or m != prev + 1):
            runs += 1
        prev = m
    return runs


def check(kvmap, b, e):
    gd = api.attn_group_desc(kvmap, b, e, D)
    rows, general = decode(gd, b, e)
    want = np.array([honoured(int(m)) for m in kvmap[b:e]], dtype=np.int64)
    np.testing.assert_array_equal(rows[~general], want[~general])
    for g in range(0, e - b, 16):
        if general[g]:
            assert runs_in(want[g:g + 16]) > 2, f"general group {g // 16} is describable"
    return gd


def test_hand_derived_words():
    m = np.full(64, -1, dtype=np.int64)
    m[0:16] = np.arange(5, 21)                # full run at arena row 5
    m[24:32] = np.arange(100, 108)            # rows 8..15 of group 1 -> 100..107
    m[32:36] = np.arange(7, 11)               # group 2: rows 0..3 -> 7..10
    m[40:42] = [3, 4]                         #          rows 8..9 -> 3..4
    m[48], m[50], m[52] = 1, 9, 20            # group 3: three runs -> general
    gd = check(m, 0, 64)
    # word = 0x80000000 | (n - 1) << 27 | r0 << 23 | l
    assert gd[0].tolist() == [0xF8000005, 0]
    assert gd[1].tolist() == [0xBC000064, 0]
    assert gd[2].tolist() == [0x98000007, 0x8C000003]
    assert gd[3].tolist() == [1, 0]


def test_groups_follow_the_range_start():
    # a range starting 8 rows into the map: group 0 is rows 8..23 of the map
    m = np.full(8 + 40, -1, dtype=np.int64)
    m[16:24] = np.arange(50, 58)  # rows 8..15 of group 0
    m[24:32] = np.arange(58, 66)  # rows 0..7 of group 1: continues the run
    gd = check(m, 8, 48)
    assert gd.shape == (4, 2)
    assert gd[0].tolist() == [0x80000000 | (7 << 27) | (8 << 23) | 50, 0]
    assert gd[1].tolist() == [0x80000000 | (7 << 27) | (0 << 23) | 58, 0]
    assert (gd[2:] == 0).all()  # rows past the end of the range describe nothing


def test_run_across_groups_and_reach():
    m = np.full(80, -1, dtype=np.int64)
    m[8:40] = np.arange(200, 232)           # a 32-row run over three groups
    m[40] = MAX_ROW                          # last honoured row
    m[41] = MAX_ROW + 1                      # past the 32-bit reach: original row
    m[42] = 2**40                            # far past it
    m[43] = -7                               # any negative entry: original row
    gd = check(m, 0, 80)
    assert gd[0].tolist() == [0x80000000 | (7 << 27) | (8 << 23) | 200, 0]
    assert gd[1].tolist() == [0xF8000000 | 208, 0]
    assert gd[2].tolist() == [0x80000000 | (7 << 27) | 224,
                              0x80000000 | (0 << 27) | (8 << 23) | MAX_ROW]


@pytest.mark.parametrize("seed", range(12))
def test_random_maps_decode_to_the_map(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(200, 3000))
    m = np.full(n, -1, dtype=np.int64)
    nxt = int(rng.integers(0, 1000))
    for _ in range(int(rng.integers(1, 40))):
        a = int(rng.integers(0, n))
        ln = int(rng.integers(1, 40))
        kind = rng.integers(0, 6)
        seg = np.arange(nxt, nxt + ln)
        if kind == 1:
            seg = seg[::-1]
        elif kind == 2:
            seg = rng.permutation(seg)
        elif kind == 3:
            seg = seg + MAX_ROW - nxt - ln // 2  # straddles the reach
        elif kind == 4:
            seg = -rng.integers(1, 5, size=ln)
        m[a:a + ln] = seg[:max(0, min(ln, n - a))]
        nxt += ln + int(rng.integers(0, 3))
    b = int(rng.integers(0, n // 3))
    e = int(rng.integers(b + 1, n + 1))
    check(m, b, e)


def test_bad_arguments():
    m = np.full(16, -1, dtype=np.int64)
    with pytest.raises(RuntimeError):
        api.attn_group_desc(m, 4, 4, D)
