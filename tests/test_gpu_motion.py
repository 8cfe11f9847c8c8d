"""GPU parity of the upstream motion producer (include/kvp_motion.h) against
oracle/farneback.py, through the C-ABI.

Tolerances (fp32 kernels with fp64 solves against the float64 oracle):
flow |error| <= 1e-4 px at the 99.9th percentile, mean <= 5e-6 px, and max
<= 5e-2 px. The max bound is loose on purpose: the update step branches on
floor(x + dx) against the last row and column (bilinear sample or R0-only
fallback), and where x + dx lands within rounding of that edge fp32 and the
oracle may branch differently, a jump the box filter spreads over one
window. Cell maps and tile change rates: within 1e-4 relative + 1e-5
absolute of the oracle applied to the same flow. Size-independent
properties are checked at the reference's full 832x480 size: a known
translation is recovered, identical frames give exactly zero flow outside
the far-border band, the pair entry point equals the clip entry point bit
for bit.
"""

import numpy as np
import pytest
import torch
from scipy import ndimage

from kvpersist import motion
from kvpersist import workloads
from oracle import farneback as fb

pytestmark = pytest.mark.gpu
DEV = "cuda"
FLOW_P999, FLOW_MEAN, FLOW_MAX = 1e-4, 5e-6, 5e-2


def _texture(h, w, seed, sigma=2.5, pad=40):
    rng = np.random.default_rng(seed)
    t = ndimage.gaussian_filter(rng.standard_normal((h + 2 * pad, w + 2 * pad)), sigma,
                                mode="wrap")
    return (t - t.mean()) / t.std(), pad


def _shifted(tex, pad, h, w, dx, dy):
    yy, xx = np.mgrid[0:h, 0:w].astype(np.float64)
    img = ndimage.map_coordinates(tex, [yy + pad - dy, xx + pad - dx], order=3, mode="wrap")
    return np.clip(np.rint(128 + 40 * img), 0, 255).astype(np.uint8)


def _flow_ok(got, want, what=""):
    e = np.abs(np.asarray(got, np.float64) - np.asarray(want, np.float64))
    mx, mean, p999 = float(e.max()), float(e.mean()), float(np.quantile(e, 0.999))
    print(f"{what}: flow error max {mx:.3e} p99.9 {p999:.3e} mean {mean:.3e} px")
    assert p999 <= FLOW_P999 and mean <= FLOW_MEAN and mx <= FLOW_MAX, (what, mx, p999, mean)


@pytest.mark.parametrize("H,W,frames", [(96, 128, 3), (256, 320, 3), (480, 832, 3)])
def test_clip_flows_match_oracle(H, W, frames):
    clip = workloads.synthetic_clip(frames, H, W, seed=H + W)
    got = motion.farneback_flows(clip).cpu().numpy()
    want = fb.farneback_clip(clip)
    assert got.shape == want.shape == (frames - 1, H, W, 2)
    _flow_ok(got, want, f"{H}x{W}")


@pytest.mark.parametrize("params", [dict(levels=0), dict(winsize=9, iterations=2),
                                    dict(poly_n=7, poly_sigma=1.5, pyr_scale=0.6, levels=2),
                                    dict(iterations=0), dict(winsize=14)])
def test_parameter_variants_match_oracle(params):
    clip = workloads.synthetic_clip(2, 128, 160, seed=7)
    got = motion.calc_optical_flow_farneback(clip[0], clip[1], **params).cpu().numpy()
    want = fb.calc_optical_flow_farneback(clip[0], clip[1], **params)
    _flow_ok(got, want, str(params))


@pytest.mark.parametrize("H,W", [(77, 101), (12, 10), (70, 130)])
def test_odd_and_minimum_sizes_match_oracle(H, W):
    """Widths that are not a multiple of 4 (byte loads), the 10-pixel minimum
    side, and coarser levels whose sides round half to even (77 x 101 ->
    38 x 50, 70 x 130 -> 35 x 65)."""
    clip = workloads.synthetic_clip(3, H, W, seed=W)
    got = motion.farneback_flows(clip).cpu().numpy()
    _flow_ok(got, fb.farneback_clip(clip), f"{H}x{W}")


def test_unaligned_pair_pointers_equal_aligned():
    """Frames at odd byte offsets of one allocation (the pair entry takes any
    two pointers) give the same flow as the aligned clip entry."""
    clip = workloads.synthetic_clip(2, 96, 128, seed=11)
    flat = torch.zeros(2 * 96 * 128 + 8, dtype=torch.uint8, device=DEV)
    a = flat[1:1 + 96 * 128].view(96, 128)
    b = flat[3 + 96 * 128:3 + 2 * 96 * 128].view(96, 128)
    a.copy_(torch.from_numpy(clip[0]))
    b.copy_(torch.from_numpy(clip[1]))
    got = motion.calc_optical_flow_farneback(a, b)
    want = motion.farneback_flows(clip)[0]
    assert torch.equal(got, want)


def test_pair_entry_equals_clip_entry_bitwise():
    clip = workloads.synthetic_clip(4, 480, 832, seed=1)
    flows = motion.farneback_flows(clip)
    dev = torch.from_numpy(clip).to(DEV)
    for p in range(3):
        one = motion.calc_optical_flow_farneback(dev[p], dev[p + 1])
        assert torch.equal(one, flows[p]), p


@pytest.mark.parametrize("dx,dy", [(1.3, -0.7), (-6.5, 4.25)])
def test_full_size_translation_is_recovered(dx, dy):
    H, W = 480, 832
    tex, pad = _texture(H, W, 3)
    a, b = _shifted(tex, pad, H, W, 0, 0), _shifted(tex, pad, H, W, dx, dy)
    flow = motion.calc_optical_flow_farneback(a, b).cpu().numpy()[24:-24, 24:-24]
    assert abs(np.median(flow[..., 0]) - dx) < 0.05 and abs(np.median(flow[..., 1]) - dy) < 0.05
    assert np.abs(flow[..., 0] - dx).mean() < 0.1 and np.abs(flow[..., 1] - dy).mean() < 0.1
    # tile change rates of a pure translation: every interior tile near |(dx, dy)|
    _, change = motion.change_rates(torch.from_numpy(
        motion.calc_optical_flow_farneback(a, b).cpu().numpy()[None]).to(DEV))
    mid = change.cpu().numpy()[0, 10:-10]
    assert np.abs(np.median(mid) - np.hypot(dx, dy)) < 0.1


def test_identical_frames_exact_zero_outside_far_band():
    H, W = 480, 832
    tex, pad = _texture(H, W, 4)
    img = _shifted(tex, pad, H, W, 0, 0)
    flow = motion.calc_optical_flow_farneback(img, img, levels=0).cpu().numpy()
    band = 3 * 7 + 1
    assert not flow[:H - band, :W - band].any()
    assert flow[-1].any() and flow[:, -1].any()
    _flow_ok(flow, fb.calc_optical_flow_farneback(img, img, levels=0), "identical frames")


def test_change_rates_match_oracle():
    rng = np.random.default_rng(5)
    flows = (rng.standard_normal((3, 480, 832, 2)) * 2).astype(np.float32)
    cells, change = motion.change_rates(torch.from_numpy(flows).to(DEV), 30, 52, 16)
    cm_o, ch_o = fb.change_rates(flows, 30, 52, 16)
    cells, change = cells.cpu().numpy(), change.cpu().numpy()
    assert change.dtype == np.float64 and change.shape == (3, 98)
    assert np.all(np.abs(cells - cm_o) <= 1e-4 * np.abs(cm_o) + 1e-5)
    assert np.all(np.abs(change - ch_o) <= 1e-4 * np.abs(ch_o) + 1e-5)
    # other grids and a tile size that leaves a short last tile
    cells, change = motion.change_rates(torch.from_numpy(flows[:1]).to(DEV), 15, 26, 7)
    cm_o, ch_o = fb.change_rates(flows[:1], 15, 26, 7)
    assert change.shape == (1, -(-390 // 7))
    assert np.all(np.abs(change.cpu().numpy() - ch_o) <= 1e-4 * np.abs(ch_o) + 1e-5)


def test_motion_trace_matches_oracle_post_processing(tmp_path):
    clip = workloads.synthetic_clip(5, 480, 832, seed=9)
    tr = motion.motion_trace(clip)
    flows = motion.farneback_flows(clip).cpu().numpy()
    _, pairs = fb.change_rates(flows, 30, 52, 16)
    change, tau, reuse = fb.trace_from_change(pairs, 50.0)
    assert tr.change.shape == (5, 98)
    assert np.all(np.abs(tr.change - change) <= 1e-4 * np.abs(change) + 1e-5)
    assert abs(tr.tau - tau) <= 1e-4 * abs(tau) + 1e-5
    assert not tr.reuse[0].any() and abs(tr.reuse[1:].mean() - 0.5) < 0.01
    csv_path, meta_path = motion.write_trace(tr, tmp_path, source="synthetic")
    lines = csv_path.read_text().splitlines()
    assert lines[0] == "frame_id,tile_id,motion_score,is_static,token_start,token_count,reuse"
    assert len(lines) == 1 + 5 * 98
    assert lines[98].split(",")[4:6] == ["1552", "8"]
    import json
    meta = json.loads(meta_path.read_text())
    assert meta["num_tiles"] == 98 and meta["grid"] == [30, 52] and meta["cell_px"] == [16, 16]
    assert meta["farneback"] == motion.FARNEBACK


def test_trace_drives_the_policy_cli(tmp_path):
    """The written trace feeds policy_experiment --motion-csv (reference
    CSV columns incl. reuse): reuse_weighted in streaming mode runs on it and
    leaves the attention output bit-identical to policy none."""
    import subprocess
    from kvpersist import _lib
    frames, tokens, hidden, heads, tt = 3, 1560, 256, 2, 16
    tr = motion.motion_trace(workloads.synthetic_clip(frames, 480, 832, seed=4))
    csv_path, _ = motion.write_trace(tr, tmp_path)
    rng = np.random.default_rng(8)
    paths = []
    for name in "qkv":
        p = tmp_path / f"{name}.bin"
        rng.standard_normal((frames * tokens, hidden), dtype=np.float32).tofile(p)
        paths.append(p)
    common = ["--attn-mode", "cross", "--q", str(paths[0]), "--k", str(paths[1]), "--v",
              str(paths[2]), "--frames", str(frames), "--tokens", str(tokens), "--hidden",
              str(hidden), "--heads", str(heads), "--tile-tokens", str(tt)]

    def run(args):
        return subprocess.run([str(_lib.CLI_PATH), *args], capture_output=True, text=True,
                              timeout=120)
    r0 = run(["--policy", "none", "--out", str(tmp_path / "none.bin"), *common])
    assert r0.returncode == 0, r0.stderr
    r1 = run(["--policy", "reuse_weighted", "--streaming", "--motion-csv", str(csv_path),
              "--out", str(tmp_path / "rw.bin"), "--set-aside-bytes", str(8 * tt * hidden * 8),
              *common])
    assert r1.returncode == 0, r1.stderr
    assert r1.stdout.splitlines()[0].startswith("policy=reuse_weighted slots=8")
    assert any(ln.startswith("streamed staged_bytes=") for ln in r1.stdout.splitlines())
    a = np.fromfile(tmp_path / "none.bin", dtype=np.float32)
    b = np.fromfile(tmp_path / "rw.bin", dtype=np.float32)
    assert a.size == frames * tokens * hidden and np.array_equal(a, b)


def test_command_line_writes_the_trace(tmp_path):
    """python -m kvpersist.motion --frames-npy clip.npy (the script's outputs:
    CSV rows and meta JSON, grid and tile size from a grounding config)."""
    import json
    import subprocess
    import sys
    clip = workloads.synthetic_clip(4, 480, 832, seed=12)
    np.save(tmp_path / "clip.npy", clip)
    cfg = tmp_path / "grounding.json"
    cfg.write_text(json.dumps({"model": {"latent_grid": [30, 52], "tile_size_tokens": 16}}))
    out = tmp_path / "traces"
    r = subprocess.run([sys.executable, "-m", "kvpersist.motion", "--frames-npy",
                        str(tmp_path / "clip.npy"), "--out-dir", str(out), "--config", str(cfg),
                        "--frames", "3"], capture_output=True, text=True, timeout=240,
                       cwd=str(motion.Path(motion.__file__).resolve().parents[1]))
    assert r.returncode == 0, r.stderr
    assert "tiles/frame: 98  rows written: 294" in r.stdout
    rows = (out / "motion_trace_real.csv").read_text().splitlines()
    assert len(rows) == 1 + 3 * 98
    meta = json.loads((out / "trace_real_meta.json").read_text())
    assert meta["frames"] == 3 and meta["size"] == [832, 480]
    assert 0.0 <= meta["reuse_fraction_achieved"] <= 1.0


def test_full_flow_clip_and_latents_to_gated_attention():
    """The reference's whole flow on the device: a clip's Farneback change
    rates (the motion producer) rank the tiles, a bf16 backbone produces
    layer K/V from latents (the K/V producer), and the motion-gated
    cross-frame pipeline stages the top-ranked tiles into the arena. The
    output equals policy none bit for bit, the arena holds tiles, and the
    attention is within the bf16 bar of the oracle."""
    from kvpersist import FramePipeline
    from kvpersist import backbone as kb
    from oracle import attention as at
    frames, T, heads = 3, 1560, 12
    D = heads * 128
    tr = motion.motion_trace(workloads.synthetic_clip(frames, 480, 832, seed=13))
    scores = tr.change.astype(np.float32)                     # [frames, 98]
    cfg = kb.BackboneConfig(num_layers=2, hidden_dim=D, num_heads=heads)
    model = kb.SelfAttentionBackbone(cfg, seed=31, dtype="bf16")
    lat = torch.randn(frames, 16, 30, 52, generator=torch.Generator(device=DEV).manual_seed(3),
                      device=DEV)
    _, k, v, q = model.forward_token_major(lat, keep_q=True)
    ql, kl, vl = q[1].contiguous(), k[1].contiguous(), v[1].contiguous()
    outs = {}
    for policy, aside in (("none", 0), ("motion", 64 * 16 * 2 * D * 2)):
        pl = FramePipeline(policy, cross=True, streaming=False, frames=frames, T=T, D=D,
                           heads=heads, tile_tokens=16, set_aside_bytes=aside, dtype=1)
        pl.set_scores(scores.reshape(-1))
        out = torch.empty_like(ql)
        pl.run(ql, kl, vl, out)
        torch.cuda.synchronize()
        if policy == "motion":
            assert pl.staged_tiles() > 0
        outs[policy] = out.cpu()
        pl.close()
    assert torch.equal(outs["none"], outs["motion"])
    want = at.attention_frames(ql.float().cpu(), kl.float().cpu(), vl.float().cpu(), frames, T,
                               heads, "cross")
    assert float((outs["none"].float() - want).abs().max()) <= 2e-2
    model.close()


def test_file_flow_backbone_bins_and_trace_drive_the_cli(tmp_path):
    """The reference's file-based flow: the motion trace CSV of a clip
    (gen_motion_from_video), one backbone layer's q/k/v exported as flat fp32
    bins (export_bins), then policy_experiment over both — motion-gated
    output bit-identical to policy none and within the fp32 bar of the
    oracle."""
    import subprocess
    from kvpersist import _lib, export_bins
    from kvpersist import backbone as kb
    from oracle import attention as at
    frames, T, heads = 3, 1560, 2
    D = heads * 128
    tr = motion.motion_trace(workloads.synthetic_clip(frames, 480, 832, seed=14))
    csv_path, _ = motion.write_trace(tr, tmp_path)
    model = kb.SelfAttentionBackbone(kb.BackboneConfig(num_layers=1, hidden_dim=D,
                                                       num_heads=heads), seed=5, dtype="fp32")
    lat = torch.randn(frames, 16, 30, 52, generator=torch.Generator(device=DEV).manual_seed(6),
                      device=DEV)
    _, k, v, q = model.forward_token_major(lat, keep_q=True)
    qp, kp, vp = export_bins.export_layer(q[0], k[0], v[0], tmp_path, "L0")
    model.close()
    common = ["--attn-mode", "cross", "--q", str(qp), "--k", str(kp), "--v", str(vp),
              "--frames", str(frames), "--tokens", str(T), "--hidden", str(D), "--heads",
              str(heads), "--tile-tokens", "16"]

    def run(args):
        return subprocess.run([str(_lib.CLI_PATH), *args], capture_output=True, text=True,
                              timeout=120)
    r0 = run(["--policy", "none", "--out", str(tmp_path / "none.bin"), *common])
    assert r0.returncode == 0, r0.stderr
    r1 = run(["--policy", "motion", "--motion-csv", str(csv_path), "--out",
              str(tmp_path / "m.bin"), "--set-aside-bytes", str(22 * 16 * D * 8), *common])
    assert r1.returncode == 0, r1.stderr
    assert r1.stdout.splitlines()[0].startswith("policy=motion slots=22")
    a = np.fromfile(tmp_path / "none.bin", dtype=np.float32).reshape(frames * T, D)
    b = np.fromfile(tmp_path / "m.bin", dtype=np.float32).reshape(frames * T, D)
    assert np.array_equal(a, b)
    qh = torch.from_numpy(np.fromfile(qp, dtype=np.float32).reshape(frames * T, D))
    kh = torch.from_numpy(np.fromfile(kp, dtype=np.float32).reshape(frames * T, D))
    vh = torch.from_numpy(np.fromfile(vp, dtype=np.float32).reshape(frames * T, D))
    want = at.attention_frames(qh, kh, vh, frames, T, heads, "cross").numpy()
    err = np.abs(a - want)
    assert err.max() <= 1e-3 and err.mean() <= 1e-4, (err.max(), err.mean())


def test_bad_arguments_raise():
    clip = workloads.synthetic_clip(2, 64, 64, seed=2)
    with pytest.raises(RuntimeError, match="flags"):
        motion.calc_optical_flow_farneback(clip[0], clip[1], flags=256)
    with pytest.raises(RuntimeError, match="winsize"):
        motion.calc_optical_flow_farneback(clip[0], clip[1], winsize=61)
    with pytest.raises(RuntimeError, match="poly_n"):
        motion.calc_optical_flow_farneback(clip[0], clip[1], poly_n=9)
    with pytest.raises(ValueError):
        motion.calc_optical_flow_farneback(clip[0], clip[1], pyr_scale=1.0)
    with pytest.raises(RuntimeError, match="grid"):
        motion.change_rates(torch.zeros(1, 64, 64, 2, device=DEV), 30, 52, 16)
    with pytest.raises(ValueError):
        motion.motion_trace(clip)                       # fewer than 3 frames
    from kvpersist import _lib
    lib = _lib.load()
    ws = torch.empty(16, dtype=torch.uint8, device=DEV)
    f = torch.from_numpy(clip).to(DEV)
    out = torch.empty(1, 64, 64, 2, device=DEV)
    rc = lib.kvp_farneback_flows(f.data_ptr(), 2, 64, 64, 0.5, 3, 15, 3, 5, 1.2, 0,
                                 ws.data_ptr(), 16, out.data_ptr(), None)
    assert rc != 0 and "workspace" in _lib.last_error()
