"""The multi-frame BASELINE configurations at their full size, through the
pipeline's layer mode (kvp_pipeline_run), one layer each.

C5: 21 frames x 3600 tokens (45 x 80 grid, 225 tiles), 12 x 128, bf16, full
causal cross-frame attention; frame 20 attends 75,600 keys and one layer's
K/V is 464 MB. Policies none and motion (sticky slots): every frame's output
bitwise equal; sampled query rows of frames 0, 10 and 20 within the bf16 bar
of the CPU oracle.

C4: 50 frames x 1560 tokens, sliding window of 8 frames, all five policies
with sticky slots: outputs bitwise equal to none on all 50 frames; sampled
rows of frames 0, 7 and 49 against the oracle over each frame's window.

The measurement harness's child (kvpersist.variance) on C4: the output
digests of none and motion agree in dense and streaming mode, and the
harness's --smoke pass runs under rocprofv3 when it is installed.
"""

import json
import shutil
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from kvpersist import BF16, FramePipeline, workloads
from oracle import attention as at

pytestmark = pytest.mark.gpu
D, H = workloads.HIDDEN, workloads.HEADS
BF16_MAX = 2e-2
ROOT = Path(__file__).resolve().parents[1]


def _run(cfg, policy, q, k, v, scores, streaming=True):
    pl = FramePipeline(policy, cross=True, streaming=streaming, frames=cfg.frames, T=cfg.tokens,
                       D=D, heads=H, tile_tokens=workloads.TILE_TOKENS,
                       set_aside_bytes=cfg.set_aside if policy != "none" else 0, dtype=BF16,
                       window_frames=cfg.window)
    pl.set_scores(scores)
    out = torch.empty_like(q)
    pl.run(q, k, v, out)
    torch.cuda.synchronize()
    staged = pl.staged_tiles()
    pl.close()
    return out, staged


def _check_rows(cfg, q, k, v, out, f, n=64):
    T = cfg.tokens
    b, e = at.key_range("cross", f, T, cfg.window)
    want = at.attention_keys(q[f * T:f * T + n].float().cpu(), k[b:e].float().cpu(),
                             v[b:e].float().cpu(), H)
    err = float((out[f * T:f * T + n].float().cpu() - want).abs().max())
    assert err <= BF16_MAX, (f, err)


def test_c5_full_size_motion_bitwise_and_oracle():
    cfg = workloads.CONFIGS["c5"]
    print(f"c5: {cfg.frames} frames x {cfg.tokens} tokens", flush=True)
    q, k, v = workloads.qkv_device(cfg.frames, cfg.tokens, seed=55, dtype=torch.bfloat16)
    scores = workloads.motion_for(cfg, 0)
    base, _ = _run(cfg, "none", q, k, v, scores)
    got, staged = _run(cfg, "motion", q, k, v, scores)
    assert staged > 0
    assert torch.equal(got, base)
    for f in (0, 10, 20):
        _check_rows(cfg, q, k, v, base, f)


def test_c4_fifty_frames_all_policies_bitwise_and_oracle():
    cfg = workloads.CONFIGS["c4"]
    print(f"c4: {cfg.frames} frames, window {cfg.window}", flush=True)
    q, k, v = workloads.qkv_device(cfg.frames, cfg.tokens, seed=44, dtype=torch.bfloat16)
    scores = workloads.motion_for(cfg, 0)
    base, _ = _run(cfg, "none", q, k, v, scores)
    for policy in ("uniform", "recency", "motion", "reuse_weighted"):
        got, staged = _run(cfg, policy, q, k, v, scores)
        assert staged > 0, policy
        assert torch.equal(got, base), policy
    for f in (0, 7, 49):
        _check_rows(cfg, q, k, v, base, f)


def _child(mode, policy, out_json):
    cmd = [sys.executable, "-m", "kvpersist.variance", "--child", mode, policy, str(out_json)]
    env = {"PYTHONPATH": str(ROOT / "cuda-kv-persistence_amd")}
    import os
    env = dict(os.environ, **env)
    subprocess.run(cmd, cwd=ROOT, env=env, check=True, timeout=240)
    return json.loads(Path(out_json).read_text())["sha256"]


def test_variance_harness_child_digests_agree(tmp_path):
    digests = {(m, p): _child(m, p, tmp_path / f"{m}_{p}.json")
               for m, p in (("dense", "none"), ("dense", "motion"), ("stream", "motion"))}
    assert len(set(digests.values())) == 1, digests


@pytest.mark.skipif(shutil.which("rocprofv3") is None, reason="rocprofv3 not installed")
def test_variance_harness_smoke_under_rocprofv3():
    import os
    env = dict(os.environ, PYTHONPATH=str(ROOT / "cuda-kv-persistence_amd"), TMPDIR="/tmp")
    res = subprocess.run([sys.executable, "-m", "kvpersist.variance", "--smoke",
                          "--timeout", "150"], cwd=ROOT, env=env, capture_output=True,
                         text=True, timeout=400)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-2000:]
    assert "Bitwise gate" in res.stdout and "PASS" in res.stdout
