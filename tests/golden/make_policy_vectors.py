"""Writes tests/golden/policy_vectors.json from the reference's own policy code.

Run in the build container (needs oracle/_ref/libref_policy.so, compiled from
/root/reference/src/tile_gating_policy.cpp by oracle/ref_build/Makefile):

    make -C oracle/ref_build && python tests/golden/make_policy_vectors.py

Each case stores how its scores are generated (seeded numpy PCG64, float32,
optionally quantised to force ties) plus a float64 checksum of the scores,
and the ids the reference implementation returns. The fixture is data only.
"""

from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
REF_LIB = ROOT / "oracle" / "_ref" / "libref_policy.so"
OUT = Path(__file__).with_name("policy_vectors.json")

POLICIES = ("none", "uniform", "recency", "motion", "reuse_weighted")


def scores_for(case: dict) -> np.ndarray:
    rng = np.random.default_rng(case["seed"])
    s = rng.random(case["n"], dtype=np.float32)
    if case.get("levels"):
        s = (np.floor(s * case["levels"]) / case["levels"]).astype(np.float32)
    if case.get("scale"):
        s = (s * np.float32(case["scale"])).astype(np.float32)
    return s


def cases() -> list[dict]:
    out = []
    seed = 1000
    for n in (1, 7, 98, 196, 784, 2450, 4900):
        for m in (0, 1, 11, 22, 98, 300):
            for levels in (0, 4):
                for tpf, total in ((98, 8), (98, 50), (7, 3)):
                    if n > 784 and (tpf, total) == (7, 3):
                        continue
                    seed += 1
                    out.append(dict(seed=seed, n=n, max=m, levels=levels, tpf=tpf,
                                    total_frames=total, scale=(4.0 if levels else 0)))
    return out


def main() -> None:
    lib = ctypes.CDLL(str(REF_LIB))
    lib.ref_policy_select.restype = ctypes.c_int
    lib.ref_policy_select.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_int,
                                      ctypes.POINTER(ctypes.c_float), ctypes.c_int, ctypes.c_int,
                                      ctypes.POINTER(ctypes.c_long)]
    records = []
    for c in cases():
        s = scores_for(c)
        sp = s.ctypes.data_as(ctypes.POINTER(ctypes.c_float))
        rec = dict(c, checksum=float(s.astype(np.float64).sum()), expected={})
        for pol in POLICIES:
            cap = max(c["max"], 1)
            buf = (ctypes.c_long * cap)()
            k = lib.ref_policy_select(pol.encode(), c["tpf"], c["total_frames"], sp, c["n"],
                                      c["max"], buf)
            rec["expected"][pol] = [int(buf[i]) for i in range(k)]
        records.append(rec)
    OUT.write_text(json.dumps({"generator": "tests/golden/make_policy_vectors.py",
                               "source": "reference src/tile_gating_policy.cpp via oracle/_ref",
                               "cases": records}, separators=(",", ":")))
    print(f"{len(records)} cases -> {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
