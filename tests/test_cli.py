"""The policy_experiment driver: the reference's flags, file formats and
output lines (reference: src/run_policy_experiment.cu:71-317).

CPU: argument errors are reported before any device work.
GPU: flat fp32 bins + motion CSV in, flat fp32 out, checked against the
oracle and policy none bit for bit, with the reference's stdout lines.
"""

import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as at

ROOT = Path(__file__).resolve().parents[1]
BIN = ROOT / "cuda-kv-persistence_amd" / "bin" / "policy_experiment"

pytestmark = pytest.mark.skipif(not BIN.exists(), reason="policy_experiment not built")


def _run(args, **kw):
    return subprocess.run([str(BIN), *args], capture_output=True, text=True, timeout=120, **kw)


@pytest.mark.parametrize("args,msg", [
    (["--bogus"], "unknown arg --bogus"),
    (["--policy"], "missing value for --policy"),
    (["--frames", "eight"], "--frames needs an integer"),
    (["--window", "3x"], "--window needs an integer"),
    (["--policy", "none", "--dtype", "fp8"], "unknown dtype fp8"),
    (["--policy", "most_recent"], "unknown policy most_recent"),
])
def test_argument_errors_exit_before_device_work(args, msg):
    r = _run(args)
    assert r.returncode == 1
    assert msg in r.stderr


def test_missing_input_file_is_reported():
    r = _run(["--policy", "none", "--q", "/nonexistent/q.bin", "--frames", "1", "--tokens", "16",
              "--hidden", "128", "--heads", "1"])
    assert r.returncode == 1 and "cannot open /nonexistent/q.bin" in r.stderr


def _write_inputs(tmp, frames, tokens, hidden, seed):
    rng = np.random.default_rng(seed)
    arrs = [rng.standard_normal((frames * tokens, hidden), dtype=np.float32) for _ in range(3)]
    paths = []
    for name, a in zip("qkv", arrs):
        p = tmp / f"{name}_t.bin"
        a.tofile(p)
        paths.append(p)
    return arrs, paths


def _write_csv(path, frames, tiles, tile_tokens, seed):
    rng = np.random.default_rng(seed)
    lines = ["frame_id,tile_id,motion_score,is_static,token_start,token_count"]
    scores = rng.random((frames, tiles), dtype=np.float32)
    for f in range(frames):
        for t in range(tiles):
            lines.append(f"{f},{t},{scores[f, t]:.6f},{int(scores[f, t] < 0.3)},"
                         f"{t * tile_tokens},{tile_tokens}")
    path.write_text("\n".join(lines) + "\n")


@pytest.mark.gpu
@pytest.mark.parametrize("streaming", [False, True])
def test_cli_cross_motion_matches_oracle_and_none(tmp_path, streaming):
    frames, tokens, hidden, heads, tt = 3, 64, 256, 2, 16
    tiles = tokens // tt
    (q, k, v), (qp, kp, vp) = _write_inputs(tmp_path, frames, tokens, hidden, seed=5)
    csv = tmp_path / "motion.csv"
    _write_csv(csv, frames, tiles, tt, seed=6)
    tile_bytes = tt * hidden * 4 * 2
    common = ["--attn-mode", "cross", "--q", str(qp), "--k", str(kp), "--v", str(vp),
              "--frames", str(frames), "--tokens", str(tokens), "--hidden", str(hidden),
              "--heads", str(heads), "--tile-tokens", str(tt)]
    out_none = tmp_path / "o_none.bin"
    r0 = _run(["--policy", "none", "--out", str(out_none), *common])
    assert r0.returncode == 0, r0.stderr
    out_m = tmp_path / "sub" / "o_motion.bin"
    args = ["--policy", "motion", "--motion-csv", str(csv), "--out", str(out_m),
            "--set-aside-bytes", str(2 * tile_bytes), *common]
    if streaming:
        args.append("--streaming")
    r1 = _run(args)
    assert r1.returncode == 0, r1.stderr
    lines = r1.stdout.splitlines()
    assert lines[0] == f"policy=motion slots=2 tile_bytes={tile_bytes} set_aside={2 * tile_bytes}"
    assert lines[1].startswith("frame 0 selected tiles:")
    assert re.fullmatch(r"frame 0 selected tiles:( \d+\(f\d+,t\d+,score \d\.\d{3}\))+", lines[1])
    if streaming:
        assert any(re.fullmatch(r"streamed staged_bytes=\d+", ln) for ln in lines)
    assert lines[-1] == f"policy=motion -> {out_m} ({frames * tokens * hidden * 4} bytes)"
    got_none = np.fromfile(out_none, dtype=np.float32).reshape(frames * tokens, hidden)
    got_m = np.fromfile(out_m, dtype=np.float32).reshape(frames * tokens, hidden)
    assert np.array_equal(got_none, got_m)
    want = at.attention_frames(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                               frames, tokens, heads, "cross").numpy()
    err = np.abs(got_m - want)
    assert err.max() <= 1e-3 and err.mean() <= 1e-4, (err.max(), err.mean())
