#!/usr/bin/env python3
"""Benchmark of the KVMap-attention + KV-arena hot path on one MI355X.

Workload "C3", the configuration of the headline metric: Wan2.1-1.3B shape,
8 frames x 1560 tokens, 12 heads x 128, 30 layers, bf16 Q/K/V ~ N(0,1)
(drawn on the device, seed 42 + layer), causal cross-frame attention, motion
scores from a seeded smooth AR(1) field. One step = the whole 30-layer pass
of the gated pipeline: per layer, every frame's policy select and arena
plan on the host, one staging launch (the shared layer arena, every
frame's KVMap slice and descriptor table), one attention launch over all 8
frames; all stream-ordered.

value = ms per query frame of that step (all 30 layers), policy `motion`
(override with --policy, workload with --config c4 / c5).

Reported per policy (none / uniform / recency / motion / reuse_weighted):
pipeline ms/frame; attention-kernel ms/frame, TFLOP/s and fraction of the
dense bf16 MFMA peak (HIP events around each layer launch, on the launch
stream, the median of 5 passes over the layers); fabric read bytes per frame of the attention kernel and of all
library kernels, their delta vs none, and GB/s with the fraction of HBM
peak. The bytes come from rocprofv3 --pmc child runs of this same script
(`--profile-policy P`), started before this process touches the GPU; each
child also runs a 256 MiB device copy whose counter readings calibrate the
scale of FETCH_SIZE / WRITE_SIZE. `roofline` is the dominant kernel's
(attn_fwd_bf16, the headline policy's instantiation). `cpu_baseline` is the
oracle's PyTorch fp32 attention on a bounded sample on this host's cores.
`c4` / `c5` objects: the other multi-frame configurations, motion policy.

The map-free kernel (policy none) and the descriptor kernel (the gated
policies) differ in fabric reads even where the descriptor kernel reads no
arena row, because their per-tile timing keeps an XCD's workgroups in step
differently. So the same quantities are also reported for policy none run
through the descriptor kernel with an empty table (`none_descriptor_kernel`),
with every gated policy's time and read delta against it (`..._same_kernel`):
the arena's own effect.

Also reported under "kv_producer": the upstream K/V producer (the reference's
DiT backbone forward, src/backbone.py:8-67) at the C3 frame set, whole
forward and per stage, each stage against its roofline. Under
"motion_producer": the upstream motion producer (the reference's Farneback
flow + per-tile change rates, traces/gen_motion_from_video.py:104-121) over a
50-frame 832x480 clip, per launch kind, the dominant kernel against the HBM
roofline.

python bench.py [--steps K] [--warmup W] [--policy P] [--config c3|c4|c5]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "cuda-kv-persistence_amd"))

METRIC = "attn ms/frame + MFMA util + HBM read bytes/frame vs policy None, Wan2.1-1.3B"
BF16_PEAK_TFLOPS = 2516.6  # MI355X dense bf16 MFMA
FP32_PEAK_TFLOPS = 157.3   # MI355X fp32 MFMA
HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--policy", default="motion")
    ap.add_argument("--layers", type=int, default=30)
    ap.add_argument("--cpu-sample-units", type=int, default=3,
                    help="frame-units of the CPU baseline sample (frames 0..1 of one layer = 3)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--streaming", action="store_true", help="sticky-slot arena mode")
    ap.add_argument("--step-mode", action="store_true",
                    help="profile child: frames one at a time (kvp_pipeline_step, the "
                         "reference driver's sequence) instead of the layer launch")
    ap.add_argument("--profile-policy", default=None,
                    help="run exactly one 30-layer step of this policy's pipeline and exit "
                         "(for rocprofv3 --pmc byte counting per policy)")
    ap.add_argument("--set-aside-tiles", type=int, default=None,
                    help="arena size in 16-token bf16 tiles (default: the configuration's "
                         "22); with --profile-policy, for the arena residency study")
    ap.add_argument("--no-producer", action="store_true",
                    help="skip the upstream K/V producer measurement")
    ap.add_argument("--producer-only", action="store_true",
                    help="measure only the upstream K/V producer (prints its object) and exit")
    ap.add_argument("--no-motion", action="store_true",
                    help="skip the upstream motion producer measurement")
    ap.add_argument("--motion-only", action="store_true",
                    help="measure only the upstream motion producer (prints its object) and exit")
    ap.add_argument("--motion-frames", type=int, default=50,
                    help="clip length of the motion producer measurement")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run 4 device-to-device copies of 256 MiB and exit (known-size "
                         "reference for FETCH_SIZE / WRITE_SIZE scaling)")
    ap.add_argument("--config", default="c3", choices=("c3", "c4", "c5"),
                    help="headline workload (default c3, the metric's configuration)")
    ap.add_argument("--calibrate", action="store_true",
                    help="with --profile-policy: end with the 256 MiB calibration copies")
    ap.add_argument("--no-counters", action="store_true",
                    help="skip the rocprofv3 --pmc child runs (fabric bytes per policy)")
    ap.add_argument("--no-legs", action="store_true", help="skip the c4 / c5 legs")
    ap.add_argument("--cold-rows-nt", action="store_true",
                    help="KVMap launches load original (non-arena) K/V rows non-temporally")
    ap.add_argument("--counter-timeout", type=int, default=240,
                    help="seconds allowed per rocprofv3 child run")
    return ap.parse_args()


def host_cpu():
    """(logical CPUs visible to this process, CPU model name)."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return n, model


def cpu_threads():
    """Threads for the CPU baselines: the CPUs this process may use, capped by
    OMP_NUM_THREADS when set (the GPU box sets it to its 16-CPU share)."""
    n, _ = host_cpu()
    try:
        n = min(n, int(os.environ.get("OMP_NUM_THREADS", n)))
    except ValueError:
        pass
    return max(1, n)


def mfma_ceiling():
    """Dense bf16 rate the matrix cores sustain on this board when they do
    nothing else (lib/libkvpprobe.so: two 256-thread workgroups per CU, four
    independent v_mfma_f32_32x32x16_bf16 chains per wave on pseudo-random
    operands, median of 5 launches of ~20 ms after a warm-up launch): the
    power-limited counterpart of the published peak. None when the probe
    library is not built."""
    import ctypes
    path = ROOT / "cuda-kv-persistence_amd" / "lib" / "libkvpprobe.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    fn = lib.kvpprobe_mfma_bf16
    fn.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_double),
                   ctypes.POINTER(ctypes.c_double)]
    fn.restype = ctypes.c_int
    tf, ms = ctypes.c_double(), ctypes.c_double()
    if fn(150000, 5, ctypes.byref(tf), ctypes.byref(ms)) != 0:
        raise RuntimeError("MFMA ceiling probe failed")
    return {"tflops": round(tf.value, 1), "frac_of_peak": round(tf.value / BF16_PEAK_TFLOPS, 4),
            "launch_ms": round(ms.value, 3),
            "kernel": "v_mfma_f32_32x32x16_bf16 only on pseudo-random bf16 operands, "
                      "2 workgroups x 4 waves per CU, 4 chains per wave"}


def cpu_baseline(cfg, units_target: int):
    """Oracle fp32 attention (reference golden restated) on host cores."""
    import numpy as np
    import torch
    sys.path.insert(0, str(ROOT))
    from oracle import attention as at
    nthreads = cpu_threads()
    torch.set_num_threads(nthreads)
    T, D, H = cfg.tokens, 1536, 12
    rng = np.random.default_rng(42)
    frames = 1
    while sum(f + 1 for f in range(frames + 1)) <= units_target:
        frames += 1
    units = sum(f + 1 for f in range(frames))
    q = at.round_bf16(torch.from_numpy(rng.standard_normal((frames * T, D), dtype=np.float32)))
    k = at.round_bf16(torch.from_numpy(rng.standard_normal((frames * T, D), dtype=np.float32)))
    v = at.round_bf16(torch.from_numpy(rng.standard_normal((frames * T, D), dtype=np.float32)))
    at.attention_keys(q[:128], k[:T], v[:T], H)  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        for f in range(frames):
            at.attention_keys(q[f * T:(f + 1) * T], k[:(f + 1) * T], v[:(f + 1) * T], H)
        times.append(time.perf_counter() - t0)
    per_unit_s = sorted(times)[1] / units
    # C3: 36 frame-units per layer, 30 layers, 8 query frames
    ms_per_frame = per_unit_s * cfg.frame_units() * cfg.layers / cfg.frames * 1e3
    nproc, model = host_cpu()
    return {"value": round(ms_per_frame, 3), "unit": "ms/frame", "cores": nthreads,
            "host_nproc": nproc, "cpu_model": model, "kind": "port",
            "sample": f"oracle fp32 torch-CPU attention, 1 layer, query frames 0..{frames - 1} "
                      f"causal ({units} frame-units of 1560x1560x12x128), median of 3, "
                      f"extrapolated x{cfg.frame_units()}/{units} units x {cfg.layers} layers "
                      f"/ {cfg.frames} frames"}


def producer_bench(args, torch, stream):
    """Upstream K/V producer (reference: src/backbone.py:8-67) at the C3 frame
    set: 8 frames x 1560 tokens, 30 layers, hidden 1536 = 12 x 128, latent
    channels 16, bf16 projections with an fp32 residual stream.

    Times the whole forward (W warmup, K timed, HIP events on the launch
    stream), then each stage of a block over the 30 layers with events around
    every launch: LayerNorm (fp32 -> bf16, HBM-bound), the three q/k/v
    projections (one launch of the grouped proj_gemm kernel, MFMA-bound),
    intra-frame attention (all 8 frames in one launch) and out_proj with the
    residual add (the grouped projection kernel, one group, accumulating)."""
    from kvpersist import api
    from kvpersist import backbone as kb

    frames, layers = 8, args.layers
    cfg = kb.BackboneConfig(num_layers=layers)
    T, D, H = cfg.tokens_per_frame, cfg.hidden_dim, cfg.num_heads
    rows = frames * T
    model = kb.SelfAttentionBackbone(cfg, seed=0, dtype="bf16")
    gen = torch.Generator(device="cuda").manual_seed(7)
    lat = torch.randn(frames, cfg.latent_channels, cfg.latent_grid_rows, cfg.latent_grid_cols,
                      device="cuda", generator=gen)
    torch.cuda.synchronize()

    def ev():
        return torch.cuda.Event(enable_timing=True)

    for _ in range(max(1, args.warmup)):
        out = model.forward_token_major(lat, stream=stream)
    torch.cuda.synchronize()
    e0, e1 = ev(), ev()
    e0.record()
    for _ in range(args.steps):
        out = model.forward_token_major(lat, stream=stream)
    e1.record()
    torch.cuda.synchronize()
    fwd_ms = e0.elapsed_time(e1) / args.steps
    hidden, kk, vv, _ = out
    finite = bool(torch.isfinite(hidden).all()) and bool(torch.isfinite(kk[-1].float()).all())
    del out, hidden, kk, vv

    # stage pass: the block's pieces on the model's own parameters
    x = torch.randn(rows, D, device="cuda", generator=gen)
    xn = torch.empty(rows, D, dtype=torch.bfloat16, device="cuda")
    q, k, v, ctx = (torch.empty_like(xn) for _ in range(4))
    P = {n: model.param_info(n)[0] for n in model.param_names()}
    api.set_stream(stream)
    stages = {"layer_norm": [], "qkv_proj": [], "attention": [], "out_proj": []}
    for rep in range(2):  # the first pass warms plans and caches, the second is measured
        for s in stages.values():
            s.clear()
        for layer in range(layers):
            b = f"blocks.{layer}."
            marks = [ev() for _ in range(5)]
            marks[0].record()
            kb.layer_norm(x, P[b + "norm.weight"], P[b + "norm.bias"], xn, stream=stream)
            marks[1].record()
            # the three row blocks of qkv_proj in one grouped launch, as the
            # backbone runs them
            kb.proj_gemm(xn, P[b + "attn.qkv_proj.weight"], P[b + "attn.qkv_proj.bias"],
                         [q, k, v], tile_n=128, stream=stream)
            marks[2].record()
            api.attn_forward_launcher_bf16(q, k, v, None, None, ctx, frames, T, D, H,
                                           remap=False)
            marks[3].record()
            kb.linear(ctx, P[b + "attn.out_proj.weight"], P[b + "attn.out_proj.bias"], x,
                      accumulate=True, stream=stream)
            marks[4].record()
            for j, name in enumerate(stages):
                stages[name].append((marks[j], marks[j + 1]))
        torch.cuda.synchronize()
    api.set_stream(None)

    def avg_ms(name):
        pairs = stages[name]
        return sum(a.elapsed_time(b) for a, b in pairs) / len(pairs)

    ln_ms, qkv_ms = avg_ms("layer_norm"), avg_ms("qkv_proj")
    att_ms, out_ms = avg_ms("attention"), avg_ms("out_proj")
    ln_bytes = rows * D * (4 + 2) + 2 * D * 4
    qkv_flops = 3 * 2 * rows * D * D
    att_flops = frames * 4 * T * T * D
    out_flops = 2 * rows * D * D

    def roof(bound, amount, ms, unit_peak, unit, what):
        ach = amount / (ms * 1e-3) / (1e9 if unit == "GB/s" else 1e12)
        return {"bound": bound, "achieved": round(ach, 2), "peak": unit_peak, "unit": unit,
                "frac": round(ach / unit_peak, 4), "avg_launch_ms": round(ms, 5),
                "per_launch": what}

    prod = {
        "metric": "K/V producer ms/frame (30-layer forward, per-layer K/V into HBM)",
        "value": round(fwd_ms / frames, 4),
        "unit": "ms/frame",
        "ms_per_forward": round(fwd_ms, 3),
        "tokens_per_s": round(rows / (fwd_ms * 1e-3)),
        "outputs_finite": finite,
        "config": {"workload": "SelfAttentionBackbone forward, 8 frames x 1560 tokens, 30 layers, "
                               "hidden 1536 (12 x 128), latent channels 16, bf16 projections, "
                               "fp32 residual stream, random-init weights (seed 0)",
                   "frames": frames, "layers": layers, "dtype": "bf16"},
        "stages_ms_per_layer": {"layer_norm": round(ln_ms, 5), "qkv_proj": round(qkv_ms, 5),
                                "attention": round(att_ms, 5), "out_proj": round(out_ms, 5)},
        "rooflines": {
            "layer_norm": roof("hbm", ln_bytes, ln_ms, HBM_PEAK_GBS, "GB/s",
                               f"{ln_bytes} B (fp32 row in, bf16 row out, {rows} rows)"),
            "qkv_proj": roof("mfma", qkv_flops, qkv_ms, BF16_PEAK_TFLOPS, "TFLOP/s",
                             f"proj_gemm_bf16_kernel, 3 groups in one launch, {qkv_flops} flop"),
            "attention": roof("mfma", att_flops, att_ms, BF16_PEAK_TFLOPS, "TFLOP/s",
                              f"attn_fwd_bf16_kernel intra-frame, {frames} frames, "
                              f"{att_flops} flop"),
            "out_proj": roof("mfma", out_flops, out_ms, BF16_PEAK_TFLOPS, "TFLOP/s",
                             f"proj_gemm_bf16_small_kernel, 1 group, fp32 residual added in the epilogue, {out_flops} flop"),
        },
    }
    if not args.no_cpu_baseline:
        prod["cpu_baseline"] = producer_cpu_baseline(model, cfg, frames, layers)
    model.close()
    return prod


def producer_cpu_baseline(model, cfg, frames, layers):
    """Oracle block (float64 LN and projections, fp32 torch attention) for one
    frame of one layer on host cores, scaled to ms per frame of the forward."""
    import numpy as np
    import torch
    sys.path.insert(0, str(ROOT))
    from oracle import backbone as ob
    nthreads = cpu_threads()
    torch.set_num_threads(nthreads)
    p = {n: model.get_param(n).numpy() for n in model.param_names()
         if n.startswith("blocks.0.")}
    T, D = cfg.tokens_per_frame, cfg.hidden_dim
    x = np.random.default_rng(0).standard_normal((T, D)).astype(np.float32)
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        ob.block_forward(x, p, 0, 1, T, cfg.num_heads, bf16=True)
        times.append(time.perf_counter() - t0)
    per_fl = sorted(times)[1]
    return {"value": round(per_fl * layers * 1e3, 3), "unit": "ms/frame", "cores": nthreads,
            "kind": "port",
            "sample": f"oracle block (LN + q/k/v projections + attention + out_proj), 1 frame x "
                      f"1 layer, median of 3, x {layers} layers"}


# Algorithmic HBM bytes per pixel of one full-size (level 0) launch, per frame
# (pyramid kinds) or per pair (flow kinds); fp32 planes, uint8 frames.
MOTION_BYTES_PER_PX = {
    "blur_rows": 1 + 4,               # uint8 frame in, fp32 row-blurred out
    "blur_cols_resize": 4 + 4,        # fp32 in, fp32 level image out
    "poly_exp": 4 + 5 * 4,            # image in, 5 expansion planes out
    "matrices_init": 2 + 5 * 4 * 2 + 5 * 4,  # coarse flow (1/4 px), R0 + R1, M out
    "box_flow": 5 * 4 + 2 * 4,        # M in, flow out
    "matrices": 2 * 4 + 5 * 4 * 2 + 5 * 4,   # flow, R0 + R1, M out
}
MOTION_PER_FRAME = ("blur_rows", "blur_cols_resize", "poly_exp")


def motion_bench(args, torch, stream):
    """Upstream motion producer (reference: traces/gen_motion_from_video.py:
    104-121) over a synthetic clip resident in HBM: --motion-frames uint8 gray
    frames of 832 x 480, Farneback(pyr_scale 0.5, levels 3, winsize 15,
    iterations 3, poly_n 5, poly_sigma 1.2) for every consecutive pair, then
    the 30 x 52 cell means and the 98 tile change rates per pair.

    Whole clip: W warmup, K timed runs (HIP events on the launch stream).
    Per launch: one run of kvp_farneback_profile (an event after every
    launch); the kind with the most time at level 0 is the dominant kernel,
    its achieved bandwidth = algorithmic bytes of one level-0 launch / its
    average level-0 duration."""
    from kvpersist import motion, workloads

    n, H, W = args.motion_frames, 480, 832
    clip = torch.from_numpy(workloads.synthetic_clip(n, H, W, seed=0)).cuda()
    flows = torch.empty(n - 1, H, W, 2, device="cuda")
    torch.cuda.synchronize()

    def run():
        motion.farneback_flows(clip, flows, stream=stream)
        return motion.change_rates(flows, 30, 52, 16, stream=stream)

    for _ in range(max(1, args.warmup)):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(args.steps):
        cells, change = run()
    e1.record()
    torch.cuda.synchronize()
    clip_ms = e0.elapsed_time(e1) / args.steps
    finite = bool(torch.isfinite(change).all())

    _, launches = motion.farneback_profile(clip, flows, stream=stream)
    per_kind, lvl0 = {}, {}
    for kind, level, ms in launches:
        per_kind[kind] = per_kind.get(kind, 0.0) + ms
        if level == 0:
            lvl0.setdefault(kind, []).append(ms)
    dominant = max(lvl0, key=lambda k: sum(lvl0[k]))
    P, pairs = H * W, n - 1

    def level0_roof(kind):
        units = n if kind in MOTION_PER_FRAME else pairs
        nbytes = MOTION_BYTES_PER_PX[kind] * P * units
        ms = sum(lvl0[kind]) / len(lvl0[kind])
        ach = nbytes / (ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(ach / HBM_PEAK_GBS, 4), "avg_launch_ms": round(ms, 5),
                "launches_per_clip": len(lvl0[kind]),
                "bytes_per_launch": nbytes,
                "per_launch": f"{MOTION_BYTES_PER_PX[kind]} B/px x {P} px x {units} "
                              f"{'frames' if kind in MOTION_PER_FRAME else 'pairs'}"}

    # fabric bytes of the level-0 launches from rocprofv3 FETCH_SIZE / WRITE_SIZE
    # runs of this workload, scaled by a copy-kernel calibration (committed)
    traffic = None
    tfile = ROOT / "profiles" / "motion_farneback_traffic.json"
    if tfile.exists():
        try:
            rec = json.loads(tfile.read_text())["kernels"].get(dominant)
            traffic = rec["hbm_bytes_per_launch"] if rec else None
        except (OSError, ValueError, KeyError):
            traffic = None
    out = {
        "metric": "motion producer ms per frame pair (Farneback flow + tile change rates)",
        "value": round(clip_ms / pairs, 5),
        "unit": "ms/pair",
        "higher_is_better": False,
        "ms_per_clip": round(clip_ms, 4),
        "pairs_per_s": round(pairs / (clip_ms * 1e-3), 1),
        "outputs_finite": finite,
        "config": {"workload": f"{n}-frame synthetic uint8 clip 832x480 (smooth texture, random "
                               f"global shift + local warp), Farneback(0.5, 3, 15, 3, 5, 1.2, 0) "
                               f"for all {pairs} pairs, 30x52 cells, 98 tiles of 16",
                   "frames": n, "dtype": "f32"},
        "launch_ms_per_clip": {k: round(v, 4) for k, v in per_kind.items()},
        "launches_per_clip": len(launches),
        "roofline": dict(level0_roof(dominant), kernel=dominant, traffic=traffic),
        "level0_rooflines": {k: level0_roof(k) for k in lvl0},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = motion_cpu_baseline(clip[:3].cpu().numpy())
    return out


def motion_cpu_baseline(frames):
    """The oracle's Farneback (numpy, float64) on a 3-frame sample of the same
    clip: both pairs, each frame's expansion computed once, as the library
    does; ms per pair."""
    sys.path.insert(0, str(ROOT))
    from oracle import farneback as fb
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        flows = fb.farneback_clip(frames)
        fb.change_rates(flows, 30, 52, 16)
        times.append(time.perf_counter() - t0)
    per_pair = sorted(times)[1] / (frames.shape[0] - 1)
    return {"value": round(per_pair * 1e3, 2), "unit": "ms/pair", "cores": 1, "kind": "port",
            "sample": f"oracle numpy Farneback + change rates, {frames.shape[0]} frames "
                      f"({frames.shape[0] - 1} pairs) of the bench clip at 832x480, median of 3 "
                      f"(the reference's cv2 path is not in this image)"}


POLICIES = ("none", "uniform", "recency", "motion", "reuse_weighted")
# Policy none run through the gated policies' kernel instantiation (group
# descriptors) with an empty table: it reads exactly the rows the map-free
# kernel reads and computes the same output, so gated policies measured
# against it show the arena's own effect on time and bytes, apart from the
# instantiation's.
SAME_KERNEL = "none_descriptor_kernel"
ATTN_KERNEL = "attn_fwd_bf16_kernel"
# a split launch's combine belongs to its attention launch (frame-by-frame
# mode only; the layer launch never splits)
COMBINE_KERNEL = "attn_combine_kernel"
STAGE_KERNELS = ("stage_kernel", "stage_runs_kernel", "map_fill_kernel", "fill_words_kernel")
COPY_KERNEL = "__amd_rocclr_copyBuffer"
CALIB_BYTES = 256 << 20
CALIB_COPIES = 4


def empty_table_launcher(torch, api, workloads, c, stream):
    """The layer launch of policy none through the descriptor instantiation
    (kvp_attn_forward_frames_gd): every KVMap entry -1, every descriptor
    entry "no arena row", a one-row arena that is never read. Returns
    launch(q, k, v, out) on `stream`."""
    F, T, W = c.frames, c.tokens, c.window
    D, H = workloads.HIDDEN, workloads.HEADS
    span = F * T
    longest = (min(W, F) if W else F) * T
    n = 4 * ((longest + 63) // 64)
    kvmap = torch.full((F * span,), -1, dtype=torch.int64, device="cuda")
    gd = torch.zeros((F * n * 2,), dtype=torch.int32, device="cuda")
    arena = torch.zeros((1, 2 * D), dtype=torch.bfloat16, device="cuda")

    def launch(q, k, v, out):
        api.attn_forward_frames_gd(q, k, v, arena, kvmap, gd, out, F, T, D, H, cross=True,
                                   window_frames=W, map_frame_stride=span, gd_frame_stride=n,
                                   stream=stream)
    return launch


def counter_run(counters, policy, args, workdir, config=None, step_mode=False, layers=None):
    """One rocprofv3 --pmc pass over `bench.py --profile-policy policy` (one
    step of that policy's pipeline plus the copy calibration) in a fresh
    child process; returns {counter: {kernel class: [per-dispatch value]}}
    (FETCH_SIZE / WRITE_SIZE in KiB). step_mode: the child runs the frames
    one at a time (kvp_pipeline_step) instead of the layer launch."""
    import csv
    import glob
    import subprocess
    config = config or args.config
    layers = layers or args.layers
    d = Path(workdir) / (f"{'_'.join(counters)}_{config}_{policy}" + ("_step" if step_mode else ""))
    cmd = ["rocprofv3", "--pmc", *counters, "--output-format", "csv", "-d", str(d), "-o", "p",
           "--", sys.executable, str(ROOT / "bench.py"), "--profile-policy", policy,
           "--config", config, "--layers", str(layers), "--steps", "1", "--calibrate"]
    if args.set_aside_tiles is not None and config == args.config:
        cmd += ["--set-aside-tiles", str(args.set_aside_tiles)]
    if args.cold_rows_nt:
        cmd.append("--cold-rows-nt")
    if args.streaming:
        cmd.append("--streaming")
    if step_mode:
        cmd.append("--step-mode")
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    proc = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=subprocess.DEVNULL,
                            stderr=subprocess.DEVNULL, start_new_session=True)
    tag = f"rocprofv3 {' '.join(counters)} {config} {policy}" + (" step" if step_mode else "")
    try:
        rc = proc.wait(timeout=args.counter_timeout)
    except subprocess.TimeoutExpired:
        os.killpg(proc.pid, 9)
        proc.wait()
        raise RuntimeError(f"{tag}: over {args.counter_timeout} s")
    per = {c: {} for c in counters}
    names = {}
    for f in glob.glob(str(d / "**" / "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                c = r["Counter_Name"]
                if c not in per:
                    continue
                key = int(r["Dispatch_Id"])
                per[c][key] = per[c].get(key, 0.0) + float(r["Counter_Value"])
                names[key] = r["Kernel_Name"]
    if not names:
        raise RuntimeError(f"{tag}: no counter rows (exit {rc})")
    res = {}
    for c in counters:
        out = {"attention": [], "staging": [], "copy": []}
        for key in sorted(per[c]):
            n = names[key]
            if ATTN_KERNEL in n or COMBINE_KERNEL in n:
                out["attention"].append(per[c][key])
            elif any(k in n for k in STAGE_KERNELS):
                out["staging"].append(per[c][key])
            elif COPY_KERNEL in n:
                out["copy"].append(per[c][key])
        res[c] = out
    if "FETCH_SIZE" in res or "WRITE_SIZE" in res:
        c0 = "FETCH_SIZE" if "FETCH_SIZE" in res else "WRITE_SIZE"
        big = [x for x in res[c0]["copy"] if x * 1024 >= CALIB_BYTES / 8]
        if len(big) != CALIB_COPIES:
            raise RuntimeError(f"{tag}: {len(big)} calibration copies")
        res[c0]["copy"] = big
    return res


def counter_set(args, work, config, policies, frames_total, *, write_policy=None,
                hit_policies=(), step_mode=False, layers=None):
    """Fabric bytes per policy of one configuration from counter_run children:
    FETCH_SIZE for every policy, WRITE_SIZE for write_policy, TCC hit rate
    for hit_policies; each scaled by its own run's calibration copies.
    Deltas are against policy none when it is among `policies`."""
    res = {"policies": {}, "runs": []}
    for pol in policies:
        r = counter_run(["FETCH_SIZE"], pol, args, work, config, step_mode, layers)["FETCH_SIZE"]
        factor = CALIB_BYTES / (sorted(r["copy"])[1] * 1024.0)
        attn = sum(r["attention"]) * 1024.0 * factor
        stage = sum(r["staging"]) * 1024.0 * factor
        res["policies"][pol] = {
            "attn_read_bytes_per_frame": round(attn / frames_total),
            "all_kernels_read_bytes_per_frame": round((attn + stage) / frames_total),
            "attn_launches": len(r["attention"]), "fetch_factor": round(factor, 4)}
        res["runs"].append(f"FETCH_SIZE {config} {pol}" + (" step" if step_mode else ""))
        log(f"counters {config}{' step' if step_mode else ''}: {pol} attention reads "
            f"{attn / frames_total / 1e9:.4f} GB/frame (calibration x{factor:.3f})")
    if write_policy:
        w = counter_run(["WRITE_SIZE"], write_policy, args, work, config, step_mode,
                        layers)["WRITE_SIZE"]
        wfactor = CALIB_BYTES / (sorted(w["copy"])[1] * 1024.0)
        res["policies"][write_policy]["attn_write_bytes_per_frame"] = round(
            sum(w["attention"]) * 1024.0 * wfactor / frames_total)
        res["policies"][write_policy]["write_factor"] = round(wfactor, 4)
        res["runs"].append(f"WRITE_SIZE {config} {write_policy}")
    for pol in hit_policies:
        h = counter_run(["TCC_HIT_sum", "TCC_MISS_sum"], pol, args, work, config, step_mode,
                        layers)
        hit, miss = sum(h["TCC_HIT_sum"]["attention"]), sum(h["TCC_MISS_sum"]["attention"])
        res["policies"][pol]["attn_l2_hit_rate"] = round(hit / max(1.0, hit + miss), 4)
        res["runs"].append(f"TCC_HIT_sum TCC_MISS_sum {config} {pol}")
    base = res["policies"].get("none")
    if base:
        for rec in res["policies"].values():
            rec["attn_read_delta_vs_none"] = round(
                rec["attn_read_bytes_per_frame"] / base["attn_read_bytes_per_frame"] - 1.0, 5)
            rec["all_kernels_read_delta_vs_none"] = round(
                rec["all_kernels_read_bytes_per_frame"]
                / base["all_kernels_read_bytes_per_frame"] - 1.0, 5)
    same = res["policies"].get(SAME_KERNEL)
    if same:
        # the arena's own effect: gated policies against none on their kernel
        for pol, rec in res["policies"].items():
            if pol not in ("none", SAME_KERNEL):
                rec["attn_read_delta_vs_none_same_kernel"] = round(
                    rec["attn_read_bytes_per_frame"] / same["attn_read_bytes_per_frame"] - 1.0,
                    5)
                rec["all_kernels_read_delta_vs_none_same_kernel"] = round(
                    rec["all_kernels_read_bytes_per_frame"]
                    / same["all_kernels_read_bytes_per_frame"] - 1.0, 5)
    return res


def measure_counters(args, cfg, headline):
    """Fabric bytes from rocprofv3 child runs, before this process touches the
    GPU: the headline configuration (every policy; WRITE_SIZE for the
    headline policy; L2 hit rate for none and it), its reference-exact
    frame-by-frame leg (none and the headline policy), and, unless --no-legs,
    C4 (every policy) and C5 (none and motion), L2 hit rate for none and
    motion."""
    import shutil
    import tempfile
    from kvpersist import workloads
    if not shutil.which("rocprofv3"):
        return {"error": "rocprofv3 not found"}
    t0 = time.perf_counter()
    out = {}
    with tempfile.TemporaryDirectory(prefix="kvp_bench_") as work:
        head = counter_set(args, work, args.config, POLICIES + (SAME_KERNEL,),
                           args.layers * cfg.frames,
                           write_policy=headline, hit_policies=("none", headline))
        out["policies"] = head["policies"]
        out["counter_runs"] = head["runs"]
        step = counter_set(args, work, args.config, ("none", headline),
                           args.layers * cfg.frames, step_mode=True)
        out["step_mode"] = step["policies"]
        out["counter_runs"] += step["runs"]
        if not args.no_legs:
            legs = {}
            for name, pols in (("c4", POLICIES + (SAME_KERNEL,)),
                               ("c5", ("none", "motion", SAME_KERNEL))):
                if name == args.config:
                    continue
                c = workloads.CONFIGS[name]
                r = counter_set(args, work, name, pols, args.layers * c.frames,
                                hit_policies=("none", "motion"))
                legs[name] = r["policies"]
                out["counter_runs"] += r["runs"]
            out["legs"] = legs
    out["seconds"] = round(time.perf_counter() - t0, 1)
    return out


def fp32_legs(torch, stream, api, FramePipeline, workloads, reps=50):
    """C1 and C2, the reference's own precision: one 1560-token frame, fp32,
    12 x 128, intra-frame attention; C1 policy none, C2 the motion-gated
    arena of 22 fp32 tiles. ms per frame (pipeline step: staging + attention)
    and the attention kernel's TFLOP/s against the fp32 MFMA peak."""
    out = {}
    for name, policy in (("c1", "none"), ("c2", "motion")):
        c = workloads.CONFIGS[name]
        T, D, H = c.tokens, workloads.HIDDEN, workloads.HEADS
        q, k, v = workloads.qkv_device(1, T, seed=42, dtype=torch.float32)
        o = torch.empty_like(q)
        pl = FramePipeline(policy, cross=False, streaming=False, frames=1, T=T, D=D, heads=H,
                           tile_tokens=workloads.TILE_TOKENS, set_aside_bytes=c.set_aside,
                           dtype=api.FP32)
        pl.set_stream(stream)
        pl.set_scores(workloads.motion_for(c) if policy != "none" else None)
        for _ in range(5):
            pl.run(q, k, v, o)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            pl.run(q, k, v, o)
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / reps
        # attention alone, the pipeline's own launch (arena region and map slice)
        gated = policy != "none"
        for rep in range(2):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(reps):
                pl.layer_attention(q, k, v, o)
            b.record()
            torch.cuda.synchronize()
        am = a.elapsed_time(b) / reps
        tf = c.flops_per_layer() / (am * 1e-3) / 1e12
        out[name] = {"workload": f"{name}: 1 frame x {T} tokens, 12 x 128, fp32, intra-frame, "
                                 f"policy {policy}" + (", arena 22 fp32 tiles" if gated else ""),
                     "pipeline_ms_per_frame": round(ms, 4),
                     "attn_kernel_ms_per_frame": round(am, 4),
                     "attn_tflops": round(tf, 2),
                     "attn_mfma_frac": round(tf / FP32_PEAK_TFLOPS, 4),
                     "peak": FP32_PEAK_TFLOPS}
        pl.close()
        log(f"leg {name}: {ms:.4f} ms/frame, attention {tf:.1f} TFLOP/s fp32")
    return out


def compulsory_read_bytes_per_frame(cfg):
    """Algorithmic read bytes of the layer launch per query frame: the launch
    reads every frame's Q rows once and, since every key row of the layer is
    in some frame's range, every K and V row once: 3 x T x D bf16 per frame."""
    return 3 * cfg.tokens * 1536 * 2


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only; --gpus must be 1 "
                                   "(multi-GPU sharding is a design note, not a code path)"}))
        sys.exit(2)
    sys.path.insert(0, str(ROOT / "cuda-kv-persistence_amd"))
    from kvpersist import workloads
    cfg = workloads.CONFIGS[args.config]
    counters = None
    child = args.profile_policy or args.copy_calibration or args.motion_only or args.producer_only
    if not child and not args.no_counters:
        # before this process initialises the GPU: the children are separate
        # processes under rocprofv3
        log("fabric-byte counters (rocprofv3 child runs) ...")
        try:
            counters = measure_counters(args, cfg, args.policy)
        except RuntimeError as e:
            counters = {"error": str(e)}
            log(f"counters failed: {e}")

    import torch
    from kvpersist import FramePipeline, _lib, api

    lib = _lib.load()
    assert torch.cuda.is_available(), "bench needs a GPU"
    dev = torch.device("cuda:0")

    def calibration_copies():
        src = torch.ones(CALIB_BYTES // 4, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(CALIB_COPIES):
            assert lib.kvp_memcpy_d2d(dst.data_ptr(), src.data_ptr(), CALIB_BYTES, None) == 0
        torch.cuda.synchronize()

    if args.copy_calibration:
        calibration_copies()
        print(json.dumps({"copy_calibration_bytes_per_copy": CALIB_BYTES,
                          "copies": CALIB_COPIES}), flush=True)
        return
    if args.motion_only:
        mot = motion_bench(args, torch, torch.cuda.current_stream().cuda_stream)
        print(json.dumps({"motion_producer": mot}), flush=True)
        return
    if args.producer_only:
        prod = producer_bench(args, torch, torch.cuda.current_stream().cuda_stream)
        print(json.dumps({"kv_producer": prod}), flush=True)
        return
    layers = args.layers
    props = torch.cuda.get_device_properties(dev)
    log(f"device {props.name} CUs={props.multi_processor_count} layers={layers}")
    stream = torch.cuda.current_stream().cuda_stream

    def workload(c):
        T, D, H, F = c.tokens, workloads.HIDDEN, workloads.HEADS, c.frames
        data = []
        for layer in range(layers):
            q, k, v = workloads.qkv_device(F, T, seed=42 + layer, dtype=torch.bfloat16,
                                           device="cuda")
            data.append((q, k, v, torch.empty_like(q), workloads.motion_for(c, layer)))
        torch.cuda.synchronize()
        return data

    def make(c, policy, set_aside):
        pl = FramePipeline(policy, cross=True, streaming=args.streaming, frames=c.frames,
                           T=c.tokens, D=workloads.HIDDEN, heads=workloads.HEADS,
                           tile_tokens=workloads.TILE_TOKENS, set_aside_bytes=set_aside,
                           dtype=api.BF16, window_frames=c.window)
        pl.set_stream(stream)
        pl.set_cold_rows_nt(args.cold_rows_nt)
        return pl

    def run_step(pl, data, step_mode=False):
        for q, k, v, out, sc in data:
            pl.set_scores(sc)
            if step_mode:
                for f in range(pl.frames):
                    pl.step(f, q, k, v, out)
            else:
                pl.run(q, k, v, out)

    def timed(pl, data, steps, step_mode=False):
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record()
        for _ in range(steps):
            run_step(pl, data, step_mode)
        e1.record()
        torch.cuda.synchronize()
        wall = (time.perf_counter() - t0) * 1e3
        return e0.elapsed_time(e1) / steps, wall / steps

    def event_passes(data, launch, passes=5):
        """HIP events around every layer's launch(q, k, v, out): one warm-up
        pass over the layers, then `passes` timed passes; returns the median
        over the passes of the mean ms per layer."""
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in data]
        scratch = torch.empty_like(data[0][3])
        per_pass = []
        for rep in range(passes + 1):
            for (q, k, v, _, _), (a, b) in zip(data, evs):
                a.record()
                launch(q, k, v, scratch)
                b.record()
            torch.cuda.synchronize()
            if rep:
                per_pass.append(sum(a.elapsed_time(b) for a, b in evs) / len(evs))
        return sorted(per_pass)[len(per_pass) // 2]

    def round_robin_passes(data, launches, passes=5):
        """event_passes for several launch(q, k, v, out) functions, their
        passes interleaved (one pass of each in turn, a warm-up pass first);
        returns {name: median over the passes of the mean ms per layer}."""
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in data]
        scratch = torch.empty_like(data[0][3])
        per = {name: [] for name in launches}
        for rep in range(passes + 1):
            for name, launch in launches.items():
                for (q, k, v, _, _), (a, b) in zip(data, evs):
                    a.record()
                    launch(q, k, v, scratch)
                    b.record()
                torch.cuda.synchronize()
                if rep:
                    per[name].append(sum(a.elapsed_time(b) for a, b in evs) / len(evs))
        return {name: sorted(v)[len(v) // 2] for name, v in per.items()}

    def attn_pass(c, pl, data, gated, passes=5):
        """The pipeline's own attention launch of every layer
        (kvp_pipeline_layer_attention, on its stream) with the layer arena,
        KVMap slices and group descriptors its last run left; ms per layer,
        the median of `passes` passes."""
        return event_passes(data, pl.layer_attention, passes)

    set_aside = (cfg.set_aside if args.set_aside_tiles is None
                 else args.set_aside_tiles * workloads.BF16_TILE_BYTES)
    data = workload(cfg)
    log(f"inputs resident ({args.config})")

    if args.profile_policy == SAME_KERNEL:
        # policy none's 30 layer launches through the descriptor
        # instantiation with an empty table, then the calibration copies
        launch = empty_table_launcher(torch, api, workloads, cfg, stream)
        for q, k, v, out, _ in data:
            launch(q, k, v, out)
        torch.cuda.synchronize()
        if args.calibrate:
            calibration_copies()
        print(json.dumps({"profile_policy": SAME_KERNEL, "config": args.config,
                          "layers": layers, "frames": cfg.frames}), flush=True)
        return
    if args.profile_policy:
        # one step (what the rocprofv3 passes count), then the calibration
        # copies; --steps > 1 also times steps 2.. (outside the profiler only)
        pl = make(cfg, args.profile_policy, set_aside)
        run_step(pl, data, args.step_mode)
        torch.cuda.synchronize()
        rec = {"profile_policy": args.profile_policy, "config": args.config,
               "step_mode": bool(args.step_mode),
               "set_aside_bytes": set_aside, "staged_tiles_last_frame": pl.staged_tiles(),
               "layers": layers, "frames": cfg.frames, "query_frames": layers * cfg.frames}
        if args.steps > 1:
            ms, _ = timed(pl, data, args.steps - 1, args.step_mode)
            rec["ms_per_frame"] = round(ms / cfg.frames, 4)
        pl.close()
        if args.calibrate:
            calibration_copies()
        print(json.dumps(rec), flush=True)
        return

    # --- headline: the policy pipeline, K timed steps ----------------------------------
    F = cfg.frames
    main_pl = make(cfg, args.policy, set_aside)
    for _ in range(args.warmup):
        run_step(main_pl, data)
    torch.cuda.synchronize()
    log(f"warmup done ({args.warmup} steps)")
    ms_step, wall_step = timed(main_pl, data, args.steps)
    log(f"policy {args.policy}: {ms_step:.3f} ms/step")

    # --- per policy: pipeline timing, bitwise gate, attention kernel alone ------------
    fl_layer = cfg.flops_per_layer()
    comp_frame = compulsory_read_bytes_per_frame(cfg)
    policies = {}
    pls = {}
    ref_out = None
    for pol in POLICIES:
        pl = main_pl if pol == args.policy else make(cfg, pol, set_aside)
        pls[pol] = pl
        run_step(pl, data)
        t, _ = timed(pl, data, max(1, min(2, args.steps)))
        o0 = data[0][3].clone()
        if ref_out is None:
            ref_out = o0
        policies[pol] = {"pipeline_ms_per_frame": round(t / F, 4),
                         "bitwise_equal_to_none": bool(torch.equal(o0, ref_out)),
                         "attn_kernel_reads_kvmap": pol != "none",
                         "staged_tiles_last_frame": pl.staged_tiles()}
        log(f"policy {pol}: {t / F:.4f} ms/frame")

    # --- the attention launch alone: every policy's own launch (its layer
    # arena and tables) and policy none through the descriptor instantiation
    # with an empty table, timed round-robin so that no policy is measured
    # later than another (the board's clock drifts over a run) --------------
    same_launch = empty_table_launcher(torch, api, workloads, cfg, stream)
    launches = {pol: pls[pol].layer_attention for pol in POLICIES}
    launches[SAME_KERNEL] = same_launch
    alone = round_robin_passes(data, launches)
    for pol in POLICIES:
        pl = pls[pol]
        lay_ms = alone[pol]
        tf = fl_layer / (lay_ms * 1e-3) / 1e12
        rec = policies[pol]
        rec.update({"attn_kernel_ms_per_frame": round(lay_ms * layers / F, 4),
                    "attn_kernel_ms_per_layer_launch": round(lay_ms, 5),
                    "attn_tflops": round(tf, 2),
                    "attn_mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4)})
        if pol != "none":
            # the layer arena: allocated once at frames x set-aside (the
            # reference's per-step arena summed over the frames), used by the
            # rows the last layer's frames map (each tile's longest prefix)
            rec["layer_arena_alloc_bytes"] = pl.layer_arena_bytes()
            rec["layer_arena_used_bytes"] = pl.layer_copied_rows() * 2 * workloads.HIDDEN * 2
            rec["layer_arena_bound_bytes"] = F * (set_aside // (2 * workloads.HIDDEN * 2)) \
                * 2 * workloads.HIDDEN * 2
        c = (counters or {}).get("policies", {}).get(pol)
        if c:
            rec.update(c)
            gbs = c["attn_read_bytes_per_frame"] * F / (lay_ms * 1e-3) / 1e9
            rec["attn_read_gbs"] = round(gbs, 1)
            rec["attn_hbm_frac"] = round(gbs / HBM_PEAK_GBS, 4)
            rec["attn_read_vs_compulsory"] = round(c["attn_read_bytes_per_frame"] / comp_frame, 4)
        if pl is not main_pl:
            pl.close()
        log(f"policy {pol}: attention alone {lay_ms * layers / F:.4f} ms/frame "
            f"({tf:.0f} TFLOP/s)")

    # policy none on the gated policies' kernel (descriptor instantiation,
    # empty table): separates the arena's own effect from the instantiation's
    same_ms = alone[SAME_KERNEL]
    same_out = torch.empty_like(data[0][3])
    same_launch(*data[0][:3], same_out)
    torch.cuda.synchronize()
    tf = fl_layer / (same_ms * 1e-3) / 1e12
    rec = {"what": "policy none through the descriptor instantiation with an empty table "
                   "(no arena row read, the map-free kernel's arithmetic)",
           "bitwise_equal_to_none": bool(torch.equal(same_out, ref_out)),
           "attn_kernel_ms_per_frame": round(same_ms * layers / F, 4),
           "attn_kernel_ms_per_layer_launch": round(same_ms, 5),
           "attn_tflops": round(tf, 2), "attn_mfma_frac": round(tf / BF16_PEAK_TFLOPS, 4)}
    c = (counters or {}).get("policies", {}).get(SAME_KERNEL)
    if c:
        rec.update(c)
        rec["attn_read_vs_compulsory"] = round(c["attn_read_bytes_per_frame"] / comp_frame, 4)
    policies[SAME_KERNEL] = rec
    for pol in POLICIES[1:]:
        policies[pol]["attn_time_delta_vs_none_same_kernel"] = round(
            policies[pol]["attn_kernel_ms_per_layer_launch"] / same_ms - 1.0, 5)
    log(f"none on the descriptor kernel: attention alone {same_ms * layers / F:.4f} ms/frame "
        f"({tf:.0f} TFLOP/s)")

    # --- reference-exact leg: the same layers frame by frame (kvp_pipeline_step:
    # the reference driver's sequence, one arena of set_aside bytes refilled per
    # frame, the reference's slot layout and KVMap values, one attention launch
    # per frame, key split + combine where a frame underfills the GPU) --------
    step_leg = {}
    step_ref = None
    for pol in ("none", args.policy):
        pl = make(cfg, pol, set_aside)
        run_step(pl, data, True)
        t, _ = timed(pl, data, max(1, min(2, args.steps)), True)
        o0 = data[0][3].clone()
        if step_ref is None:
            step_ref = o0
        step_leg[pol] = {"pipeline_ms_per_frame": round(t / F, 4),
                         "bitwise_equal_to_none": bool(torch.equal(o0, step_ref)),
                         "arena_bytes": set_aside if pol != "none" else 0}
        c = (counters or {}).get("step_mode", {}).get(pol)
        if c:
            step_leg[pol].update(c)
        pl.close()
        log(f"step mode {pol}: {t / F:.4f} ms/frame")
    step_leg["workload"] = (f"{args.config} frame by frame (kvp_pipeline_step): the reference "
                            f"driver's per-frame sequence on one {set_aside:,}-byte arena")

    head = policies[args.policy]
    lay_ms = head["attn_kernel_ms_per_layer_launch"]
    achieved = fl_layer / (lay_ms * 1e-3) / 1e12
    traffic = None
    if head.get("attn_write_bytes_per_frame") is not None:
        traffic = round((head["attn_read_bytes_per_frame"] + head["attn_write_bytes_per_frame"])
                        * F)

    # --- other multi-frame configurations (motion policy) --------------------------
    legs = {}
    if not args.no_legs:
        legs.update(fp32_legs(torch, stream, api, FramePipeline, workloads))
        for name in ("c3", "c4", "c5"):
            if name == args.config:
                continue
            c = workloads.CONFIGS[name]
            data_leg = workload(c)
            pl = make(c, "motion", c.set_aside)
            run_step(pl, data_leg)
            t, _ = timed(pl, data_leg, 2)
            # attention alone: the median of 3 passes over every layer (C5,
            # 0.5 s a launch: over the first 10 layers)
            lm = attn_pass(c, pl, data_leg[:10] if name == "c5" else data_leg, True, passes=3)
            tfl = c.flops_per_layer() / (lm * 1e-3) / 1e12
            # policy none on the same instantiation (empty table), first 10 layers
            lm_same = event_passes(data_leg[:10], empty_table_launcher(
                torch, api, workloads, c, stream), passes=3)
            nb = FramePipeline("none", cross=True, streaming=False, frames=c.frames,
                               T=c.tokens, D=workloads.HIDDEN, heads=workloads.HEADS,
                               dtype=api.BF16, window_frames=c.window)
            nb.set_stream(stream)
            o_motion = data_leg[0][3].clone()
            q, k, v, out, _ = data_leg[0]
            nb.run(q, k, v, out)
            torch.cuda.synchronize()
            legs[name] = {
                "workload": f"{name}: {c.frames} frames x {c.tokens} tokens, 12 x 128, "
                            f"{layers} layers, bf16, causal"
                            + (f", window {c.window} frames" if c.window else "")
                            + ", motion policy, arena 22 tiles",
                "pipeline_ms_per_frame": round(t / c.frames, 4),
                "attn_kernel_ms_per_frame": round(lm * layers / c.frames, 4),
                "attn_tflops": round(tfl, 2), "attn_mfma_frac": round(tfl / BF16_PEAK_TFLOPS, 4),
                "none_same_kernel_attn_ms_per_frame": round(lm_same * layers / c.frames, 4),
                "attn_time_delta_vs_none_same_kernel": round(lm / lm_same - 1.0, 5),
                "attn_launches_per_layer": 1, "key_splits": 1,
                "bitwise_equal_to_none_layer0": bool(torch.equal(o_motion, out)),
                "layer_arena_alloc_bytes": pl.layer_arena_bytes(),
                "layer_arena_used_bytes": pl.layer_copied_rows() * 2 * workloads.HIDDEN * 2}
            leg_counters = (counters or {}).get("legs", {}).get(name)
            if leg_counters:
                comp = compulsory_read_bytes_per_frame(c)
                for rec in leg_counters.values():
                    rec["attn_read_vs_compulsory"] = round(
                        rec["attn_read_bytes_per_frame"] / comp, 4)
                legs[name]["fabric_reads_per_policy"] = leg_counters
            nb.close()
            pl.close()
            del data_leg
            torch.cuda.empty_cache()
            log(f"leg {name}: {t / c.frames:.4f} ms/frame, {tfl:.0f} TFLOP/s")

    ceiling = mfma_ceiling()
    if ceiling:
        log(f"matrix-core ceiling {ceiling['tflops']} TFLOP/s "
            f"({ceiling['frac_of_peak']:.3f} of the published peak)")

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        cpu = cpu_baseline(cfg, args.cpu_sample_units)
        log(f"cpu baseline {cpu['value']} ms/frame on {cpu['cores']} cores")

    prod = None
    if not args.no_producer:
        log("upstream K/V producer ...")
        prod = producer_bench(args, torch, stream)
        log(f"producer {prod['value']} ms/frame")
    mot = None
    if not args.no_motion:
        mot = motion_bench(args, torch, stream)
        log(f"motion producer {mot['value']} ms/pair")

    value = ms_step / F
    line = {
        "metric": METRIC,
        "value": round(value, 4),
        "unit": "ms/frame",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (device N(0,1) Q/K/V, seeded motion field)",
        "config": {
            "workload": f"{args.config}: causal cross-frame attention, {F} frames x "
                        f"{cfg.tokens} tokens, 12 heads x 128, {layers} layers, bf16, "
                        + (f"window {cfg.window} frames, " if cfg.window else "")
                        + f"KVMap arena {set_aside // workloads.BF16_TILE_BYTES} tiles "
                          f"({set_aside:,} B)",
            "policy": args.policy, "streaming": bool(args.streaming),
            "cold_rows_nt": bool(args.cold_rows_nt), "frames": F,
            "tokens_per_frame": cfg.tokens, "heads": workloads.HEADS, "head_dim": 128,
            "layers": layers, "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "mfma",
            "kernel": ("attn_fwd_bf16_kernel, " +
                       ("KVMap instantiation" if head["attn_kernel_reads_kvmap"]
                        else "map-free instantiation") +
                       f", one launch per layer ({F} frames)"),
            "achieved": round(achieved, 2),
            "peak": BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / BF16_PEAK_TFLOPS, 4),
            "traffic": traffic,
            "flops_per_launch": round(fl_layer),
            "avg_launch_ms": lay_ms,
            "compulsory_read_bytes_per_launch": round(comp_frame * F),
            "compulsory_write_bytes_per_launch": round(F * cfg.tokens * 1536 * 2),
            "mfma_ceiling": ceiling,
            "frac_of_ceiling": (round(achieved / ceiling["tflops"], 4) if ceiling else None),
        },
        "cpu_baseline": cpu,
        "policies": policies,
        "reference_exact_step_mode": step_leg,
        "counters": ({k: v for k, v in counters.items()
                      if k not in ("policies", "step_mode", "legs")}
                     if counters else None),
        "legs": legs,
        "wall_ms_per_step": round(wall_step, 3),
        "kv_producer": prod,
        "motion_producer": mot,
    }
    print(json.dumps(line), flush=True)
    main_pl.close()


if __name__ == "__main__":
    main()
