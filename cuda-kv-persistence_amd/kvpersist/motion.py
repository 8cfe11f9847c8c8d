"""Python mirror of the upstream motion producer, over the C-ABI of include/kvp_motion.h.

The reference turns a clip into the motion trace the policies read
(reference: traces/gen_motion_from_video.py): Farneback flow between
consecutive gray frames (:104-111), the flow magnitude averaged over 16x16
pixel latent-grid cells (:61-67,112-113) and over row-major 16-cell tiles
(:114-120), frame 0 borrowing frame 1's rates (:121), the reuse threshold tau
= a percentile of the rates of frames 1.. (:123-125), then
``motion_trace_real.csv`` and ``trace_real_meta.json`` (:127-186).

Here the flow, the cells and the tile rates run in libkvpersist.so on the
device (one pass over the whole clip); the percentile, the CSV and the meta
statistics are the same small host steps as the reference's. Frame decoding,
BGR->gray and the INTER_AREA resize to 832x480 (:37-58) and the heat-map PNG
need OpenCV and stay outside: frames enter as uint8 gray arrays already at
the grid's pixel size (``--frames-npy``).

    flow = calc_optical_flow_farneback(prev, next, None, 0.5, 3, 15, 3, 5, 1.2, 0)
    trace = motion_trace(frames_u8)      # frames [n, 480, 832] uint8
    write_trace(trace, "traces", source="clip")
"""

from __future__ import annotations

import argparse
import csv
import json
import sys
from dataclasses import dataclass, field
from datetime import date
from pathlib import Path

import numpy as np
import torch

from . import _lib
from .api import _check, _ptr

# reference: traces/gen_motion_from_video.py:107-108
FARNEBACK = dict(pyr_scale=0.5, levels=3, winsize=15, iterations=3, poly_n=5, poly_sigma=1.2,
                 flags=0)

# One workspace per device, shared by every call there: calls that overlap on
# different streams of one device race on it.
_workspaces: dict[int, torch.Tensor] = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-device workspace, grown on demand (calls on one device share it)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = _workspaces.get(idx)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        _workspaces[idx] = ws
    return ws


def _frames_u8(x, device=None) -> torch.Tensor:
    if isinstance(x, np.ndarray):
        x = torch.from_numpy(np.ascontiguousarray(x))
    if x.dtype != torch.uint8:
        raise ValueError("frames must be uint8 gray images")
    if not x.is_cuda:
        x = x.to(device or "cuda")
    return x.contiguous()


def _params(kw) -> dict:
    p = dict(FARNEBACK)
    unknown = set(kw) - set(p)
    if unknown:
        raise TypeError(f"unknown Farneback parameters {sorted(unknown)}")
    p.update(kw)
    return p


def farneback_flows(frames, flows: torch.Tensor | None = None, stream: int | None = None,
                    **params) -> torch.Tensor:
    """Flow of every consecutive pair of a clip: frames uint8 [n, H, W] ->
    fp32 [n-1, H, W, 2] on the device, pair p = (frames[p], frames[p+1])."""
    fr = _frames_u8(frames)
    if fr.dim() != 3:
        raise ValueError("frames must be [n, H, W]")
    n, H, W = fr.shape
    p = _params(params)
    lib = _lib.load()
    need = lib.kvp_farneback_workspace_bytes(n, W, H, float(p["pyr_scale"]), int(p["levels"]))
    if need < 0:
        raise ValueError(f"bad clip shape {tuple(fr.shape)} or pyramid parameters {p}")
    ws = _workspace(fr.device, need)
    if flows is None:
        flows = torch.empty(n - 1, H, W, 2, dtype=torch.float32, device=fr.device)
    elif flows.shape != (n - 1, H, W, 2) or flows.dtype != torch.float32:
        raise ValueError("flows must be float32 [n-1, H, W, 2]")
    _check(lib.kvp_farneback_flows(_ptr(fr), n, W, H, float(p["pyr_scale"]), int(p["levels"]),
                                   int(p["winsize"]), int(p["iterations"]), int(p["poly_n"]),
                                   float(p["poly_sigma"]), int(p["flags"]), _ptr(ws),
                                   ws.numel(), _ptr(flows), stream), "kvp_farneback_flows")
    return flows


KINDS = ("blur_rows", "blur_cols_resize", "poly_exp", "matrices_init", "box_flow", "matrices")


def farneback_profile(frames, flows: torch.Tensor | None = None, stream: int | None = None,
                      **params):
    """farneback_flows with an event after every launch (synchronises):
    -> (flows, [(kind name, pyramid level, ms), ...] in launch order)."""
    fr = _frames_u8(frames)
    n, H, W = fr.shape
    p = _params(params)
    lib = _lib.load()
    need = lib.kvp_farneback_workspace_bytes(n, W, H, float(p["pyr_scale"]), int(p["levels"]))
    if need < 0:
        raise ValueError(f"bad clip shape {tuple(fr.shape)} or pyramid parameters {p}")
    ws = _workspace(fr.device, need)
    if flows is None:
        flows = torch.empty(n - 1, H, W, 2, dtype=torch.float32, device=fr.device)
    cap = 1024
    ms = np.zeros(cap, dtype=np.float32)
    kind = np.zeros(cap, dtype=np.int32)
    level = np.zeros(cap, dtype=np.int32)
    count = np.zeros(1, dtype=np.int32)
    _check(lib.kvp_farneback_profile(_ptr(fr), n, W, H, float(p["pyr_scale"]), int(p["levels"]),
                                     int(p["winsize"]), int(p["iterations"]), int(p["poly_n"]),
                                     float(p["poly_sigma"]), int(p["flags"]), _ptr(ws),
                                     ws.numel(), _ptr(flows), ms.ctypes.data, kind.ctypes.data,
                                     level.ctypes.data, cap, count.ctypes.data, stream),
           "kvp_farneback_profile")
    k = int(count[0])
    return flows, [(KINDS[kind[i]], int(level[i]), float(ms[i])) for i in range(k)]


def calc_optical_flow_farneback(prev, next, flow=None, pyr_scale=0.5, levels=3, winsize=15,
                                iterations=3, poly_n=5, poly_sigma=1.2, flags=0,
                                stream: int | None = None) -> torch.Tensor:
    """cv2.calcOpticalFlowFarneback's argument order and meaning; prev/next
    uint8 [H, W] -> flow fp32 [H, W, 2] (dx, dy) on the device. A given
    ``flow`` tensor receives the result (flags must be 0: no initial flow)."""
    a = _frames_u8(prev)
    b = _frames_u8(next, a.device)
    if a.shape != b.shape or a.dim() != 2:
        raise ValueError("prev and next must be uint8 [H, W] of one size")
    H, W = a.shape
    lib = _lib.load()
    need = lib.kvp_farneback_workspace_bytes(2, W, H, float(pyr_scale), int(levels))
    if need < 0:
        raise ValueError(f"bad frame size {W}x{H} or pyramid parameters")
    ws = _workspace(a.device, need)
    if flow is None:
        flow = torch.empty(H, W, 2, dtype=torch.float32, device=a.device)
    _check(lib.kvp_farneback_flow(_ptr(a), _ptr(b), _ptr(flow), W, H, float(pyr_scale),
                                  int(levels), int(winsize), int(iterations), int(poly_n),
                                  float(poly_sigma), int(flags), _ptr(ws), ws.numel(), stream),
           "kvp_farneback_flow")
    return flow


def change_rates(flows: torch.Tensor, grid_rows: int = 30, grid_cols: int = 52,
                 tile_tokens: int = 16, stream: int | None = None):
    """flows fp32 [P, H, W, 2] -> (cell maps fp32 [P, rows, cols], change fp64 [P, tiles])."""
    if flows.dim() == 3:
        flows = flows.unsqueeze(0)
    P, H, W, _ = flows.shape
    tiles = -(-(grid_rows * grid_cols) // tile_tokens)
    fl = flows.contiguous()
    cells = torch.empty(P, grid_rows, grid_cols, dtype=torch.float32, device=flows.device)
    change = torch.empty(P, tiles, dtype=torch.float64, device=flows.device)
    _check(_lib.load().kvp_motion_change_rates(_ptr(fl), P, W, H, grid_rows,
                                               grid_cols, tile_tokens, _ptr(cells), _ptr(change),
                                               stream), "kvp_motion_change_rates")
    return cells, change


@dataclass
class MotionTrace:
    """The reference's per-clip results (gen_motion_from_video.py:104-126)."""
    change: np.ndarray            # [n, tiles] float64, row 0 = row 1
    tau: float
    reuse: np.ndarray             # [n, tiles] int64, row 0 = 0
    cell_maps: np.ndarray         # [n, rows, cols], row 0 zero
    tokens_per_frame: int
    tile_tokens: int
    reuse_percentile: float
    farneback: dict = field(default_factory=lambda: dict(FARNEBACK))
    size: tuple = (0, 0)          # (width, height)


def trace_from_change(change_pairs: np.ndarray, reuse_percentile: float = 50.0):
    """[n-1, tiles] pair rates -> (change [n, tiles], tau, reuse [n, tiles])
    (reference: gen_motion_from_video.py:121-126)."""
    n = change_pairs.shape[0] + 1
    change = np.zeros((n, change_pairs.shape[1]), dtype=np.float64)
    change[1:] = change_pairs
    change[0] = change[1]
    tau = float(np.percentile(change[1:], reuse_percentile))
    reuse = (change < tau).astype(np.int64)
    reuse[0] = 0
    return change, tau, reuse


def motion_trace(frames, grid=(30, 52), tile_tokens: int = 16, reuse_percentile: float = 50.0,
                 **farneback) -> MotionTrace:
    """Clip uint8 [n, H, W] (n >= 3) -> MotionTrace, flow and rates on the device."""
    fr = _frames_u8(frames)
    n = fr.shape[0]
    if n < 3:
        raise ValueError(f"need >=3 frames, got {n}")   # reference :101
    p = _params(farneback)
    flows = farneback_flows(fr, **p)
    cells, change = change_rates(flows, grid[0], grid[1], tile_tokens)
    torch.cuda.synchronize(fr.device)
    change, tau, reuse = trace_from_change(change.cpu().numpy(), reuse_percentile)
    cm = np.zeros((n,) + tuple(grid))
    cm[1:] = cells.cpu().numpy()
    return MotionTrace(change, tau, reuse, cm, grid[0] * grid[1], tile_tokens, reuse_percentile,
                       p, (fr.shape[2], fr.shape[1]))


def trace_rows(trace: MotionTrace):
    """CSV rows frame_id,tile_id,motion_score,is_static,token_start,token_count,reuse
    (reference: gen_motion_from_video.py:138-149)."""
    n, tiles = trace.change.shape
    tt, T = trace.tile_tokens, trace.tokens_per_frame
    rows = []
    for f in range(n):
        for t in range(tiles):
            cnt = tt if t < tiles - 1 else T - (tiles - 1) * tt
            rows.append([f, t, f"{trace.change[f, t]:.6f}", int(trace.change[f, t] < trace.tau),
                         t * tt, int(cnt), int(trace.reuse[f, t])])
    return rows


def read_trace_csv(path) -> np.ndarray:
    """motion_score column of a trace CSV -> float32 [frames, tiles], parsed
    as the reference's driver does (%f into a float; reference:
    src/run_policy_experiment.cu:45-69)."""
    rows = []
    with open(path, newline="") as fh:
        r = csv.reader(fh)
        next(r)                                    # header
        for rec in r:
            if rec:
                rows.append((int(rec[0]), int(rec[1]), np.float32(rec[2])))
    frames = max(f for f, _, _ in rows) + 1
    tiles = max(t for _, t, _ in rows) + 1
    out = np.zeros((frames, tiles), dtype=np.float32)
    for f, t, v in rows:
        out[f, t] = v
    return out


def trace_meta(trace: MotionTrace, source: str = "") -> dict:
    """The reference's provenance and validation block (gen_motion_from_video.py:154-176)."""
    grid = trace.cell_maps.shape[1:]
    med = np.median(trace.cell_maps[1:], axis=0)
    corr_h = float(np.corrcoef(med[:, :-1].ravel(), med[:, 1:].ravel())[0, 1])
    corr_v = float(np.corrcoef(med[:-1, :].ravel(), med[1:, :].ravel())[0, 1])
    rng = np.random.default_rng(7)
    sh = med.reshape(-1).copy()
    rng.shuffle(sh)
    sh = sh.reshape(grid)
    corr_ctrl = float(np.corrcoef(sh[:, :-1].ravel(), sh[:, 1:].ravel())[0, 1])
    w, h = trace.size
    return {
        "generated_on": date.today().isoformat(),
        "generator": "kvpersist.motion",
        "source": source, "frames": int(trace.change.shape[0]), "size": [w, h],
        "cell_px": [h // grid[0], w // grid[1]],
        "grid": [int(grid[0]), int(grid[1])], "tile_size_tokens": trace.tile_tokens,
        "num_tiles": int(trace.change.shape[1]),
        "farneback": trace.farneback,
        "tau_reuse": round(trace.tau, 6),
        "reuse_percentile_target": trace.reuse_percentile,
        "reuse_fraction_achieved": round(float(trace.reuse[1:].mean()), 4),
        "change_rate_percentiles": {
            q: round(float(np.percentile(trace.change[1:], q)), 4) for q in (10, 25, 50, 75, 90)},
        "spatial_coherence_adjacent_cell_corr": {
            "horizontal": round(corr_h, 4), "vertical": round(corr_v, 4),
            "shuffled_control": round(corr_ctrl, 4)},
    }


def write_trace(trace: MotionTrace, out_dir, source: str = "") -> tuple[Path, Path]:
    """motion_trace_real.csv + trace_real_meta.json (reference names and columns)."""
    out = Path(out_dir)
    out.mkdir(parents=True, exist_ok=True)
    csv_path = out / "motion_trace_real.csv"
    with open(csv_path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(["frame_id", "tile_id", "motion_score", "is_static", "token_start",
                    "token_count", "reuse"])
        w.writerows(trace_rows(trace))
    meta = trace_meta(trace, source)
    meta["files"] = {"csv": str(csv_path)}
    meta_path = out / "trace_real_meta.json"
    meta_path.write_text(json.dumps(meta, indent=2))
    return csv_path, meta_path


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--frames-npy", required=True,
                    help="uint8 gray clip [n, H, W] (.npy), H x W divisible by the latent grid")
    ap.add_argument("--frames", type=int, default=128, help="max frames to use")
    ap.add_argument("--reuse-percentile", type=float, default=50.0,
                    help="percentile of change-rate used as reuse threshold")
    ap.add_argument("--out-dir", default="traces")
    ap.add_argument("--config", default=None,
                    help="grounding config JSON (its model block gives the grid and tile size)")
    args = ap.parse_args(argv)
    grid, tt = (30, 52), 16
    if args.config:
        m = json.loads(Path(args.config).read_text())["model"]
        grid, tt = tuple(m["latent_grid"]), int(m["tile_size_tokens"])
    clip = np.load(args.frames_npy, allow_pickle=False)[:args.frames]
    trace = motion_trace(clip, grid=grid, tile_tokens=tt, reuse_percentile=args.reuse_percentile)
    csv_path, meta_path = write_trace(trace, args.out_dir, source=args.frames_npy)
    meta = json.loads(meta_path.read_text())
    print(f"source: {args.frames_npy} -> {clip.shape[0]} frames @ {clip.shape[2]}x{clip.shape[1]}")
    print(f"tiles/frame: {trace.change.shape[1]}  rows written: {trace.change.size}")
    print(f"change-rate percentiles (px/frame): {meta['change_rate_percentiles']}")
    print(f"tau_reuse={trace.tau:.4f} -> reuse fraction {meta['reuse_fraction_achieved']} "
          f"(target {args.reuse_percentile}%)")
    print(f"csv -> {csv_path}  meta -> {meta_path}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
