"""Flat fp32 trace binaries for the policy_experiment CLI.

The reference's `traces/export_bins.py:15-31` writes the Q, K and V arrays of
an .npz trace as raw float32 files `{q,k,v}_{stem}.bin` (row-major, no
header; shapes travel as CLI flags). `export_arrays` and the command line
below do the same; `export_layer` writes one layer of the K/V producer
(token-major [frames * T, D], any dtype, widened to fp32) in that format, so
the producer's K/V feed `policy_experiment --q --k --v` directly.

    python -m kvpersist.export_bins --npz traces/qkv_8f.npz --stem 8f --out-dir traces
"""

from __future__ import annotations

import argparse
from pathlib import Path

import numpy as np


def export_arrays(arrays, out_dir, stem: str) -> list[Path]:
    """arrays: mapping with Q, K, V (numpy or torch) -> [q, k, v] bin paths."""
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    paths = []
    for name in ("Q", "K", "V"):
        a = arrays[name]
        if hasattr(a, "detach"):                   # torch tensor (any device / dtype)
            a = a.detach().float().cpu().numpy()
        arr = np.ascontiguousarray(a, dtype=np.float32)
        p = out / f"{name.lower()}_{stem}.bin"
        arr.tofile(p)
        paths.append(p)
    return paths


def export_layer(q, k, v, out_dir, stem: str) -> list[Path]:
    """One layer's token-major q, k, v of the K/V producer -> {q,k,v}_{stem}.bin."""
    return export_arrays({"Q": q, "K": k, "V": v}, out_dir, stem)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--npz", default="traces/qkv_8f.npz")
    ap.add_argument("--stem", default="8f")
    ap.add_argument("--out-dir", default="traces")
    args = ap.parse_args(argv)
    with np.load(args.npz, allow_pickle=False) as data:
        paths = export_arrays({n: data[n] for n in ("Q", "K", "V")}, args.out_dir, args.stem)
    for name, p in zip("QKV", paths):
        n = p.stat().st_size
        print(f"{name} {n // 4} float32 -> {p} ({n} bytes)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
