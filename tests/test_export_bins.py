"""The flat fp32 trace binaries (reference: traces/export_bins.py:15-31) on the CPU."""

import subprocess
import sys

import numpy as np
import torch

from kvpersist import export_bins


def test_npz_to_bins_round_trip(tmp_path):
    rng = np.random.default_rng(1)
    q = rng.standard_normal((2 * 16, 64)).astype(np.float64)     # widened to fp32 on export
    k = rng.standard_normal((2 * 16, 64)).astype(np.float32)
    v = rng.standard_normal((2 * 16, 64)).astype(np.float32)
    np.savez(tmp_path / "qkv.npz", Q=q, K=k, V=v)
    r = subprocess.run([sys.executable, "-m", "kvpersist.export_bins", "--npz",
                        str(tmp_path / "qkv.npz"), "--stem", "t", "--out-dir", str(tmp_path / "o")],
                       capture_output=True, text=True, timeout=120,
                       cwd=str(export_bins.Path(export_bins.__file__).resolve().parents[1]))
    assert r.returncode == 0, r.stderr
    for name, a in (("q", q), ("k", k), ("v", v)):
        p = tmp_path / "o" / f"{name}_t.bin"
        assert p.stat().st_size == a.size * 4
        assert np.array_equal(np.fromfile(p, dtype=np.float32), a.astype(np.float32).ravel())


def test_export_layer_widens_bf16_tensors(tmp_path):
    t = torch.randn(48, 128).to(torch.bfloat16)
    paths = export_bins.export_layer(t, t * 2, t * 3, tmp_path, "L1")
    assert [p.name for p in paths] == ["q_L1.bin", "k_L1.bin", "v_L1.bin"]
    got = np.fromfile(paths[1], dtype=np.float32).reshape(48, 128)
    assert np.array_equal(got, (t * 2).float().numpy())
