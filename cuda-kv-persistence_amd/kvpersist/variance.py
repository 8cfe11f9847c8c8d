"""Run-to-run spread and policy separation of fabric read bytes.

Restates the reference's variance study (reference: tests/test_variance.py:1-240)
on MI355X with rocprofv3 counters instead of Nsight Compute, on two shapes
(`--shape`):

* `c4`: 50 query frames of 1560 tokens, causal
  cross-frame attention over a sliding window of 8 frames, 12 heads x 128,
  bf16, arena budget 22 bf16 tiles; combos {dense (arena), stream (sticky
  slots)} x {none, uniform, recency, motion, reuse_weighted} (the
  reference's `COMBOS`, :153-155, plus uniform, the fifth policy of its
  policy file);
* `dense50` (the shape of the reference's published scoreboard,
  docs/results/freeze_scoreboard.md:9-35, tests/test_policy_variants.py:
  209-222): 50 query frames of 1560 tokens, fp32, full causal prefix (frame
  f attends every key of frames 0..f), 12 heads x 128, set-aside 2,162,688 B
  = 11 fp32 tiles (the reference driver's slot count for its RTX 3060
  carve-out, src/run_policy_experiment.cu:143-144); combos {dense, stream} x
  {none, recency, motion, reuse_weighted}, the reference's own four;
* both: one layer, one attention launch per frame (kvp_pipeline_step, as the
  reference's `policy_experiment`), synthetic device N(0,1) Q/K/V (seed 42)
  and, unless `--motion-csv` gives a trace, the synthetic C4 motion field
  (50 x 98 tiles, camera-pan drift; `workloads.motion_for`) — the
  reference's scoreboard used its real-video trace, which needs OpenCV and a
  download;
* each frame is one attention launch (kvp_pipeline_step: frame by frame on
  one arena, the reference driver's sequence), so the launch window below
  counts frames as the reference's does; a frame whose launch splits its key
  range also runs a combine launch, counted with it (the reference's kernel
  has no split);
* each run profiles the attention launches of the run; the window is
  launches SKIP..SKIP+COUNT-1 = 34..49 (reference :39);
* metric: L2->fabric read bytes per window (`FETCH_SIZE`, KiB, scaled by the
  copy-kernel calibration of profiles/attn_bf16_c3_traffic.json) — MI355X
  exposes no Infinity-Cache hit counter, so this is the upper bound on HBM
  reads that plays the role of the reference's `dram__bytes_read.sum`; L2
  hit rate from `TCC_HIT_sum` / `TCC_MISS_sum` in a second, separate pass
  (the two counter sets together exceed the TCC block's four counters);
* REPEATS = 3 with ABBA-interleaved order across repeats (reference :160);
* bitwise gate: every gated policy's output equals policy none's of the same
  mode and repeat (compared by SHA-256 of the output bytes);
* verdicts: spread = (max - min) / median per combo, PASS <= 10 %
  (reference :41, :196-199); launches with > 20 % range across repeats
  (:206-212); policy deltas vs none and band overlap, and reuse_weighted vs
  recency band separation per mode (:214-236).

The reference locks clocks (`ncu --clock-control base`); an ordinary user
cannot pin MI355X clocks, and fabric bytes do not depend on the clock.

Usage on the GPU box, from the repository root:

    python3 -m kvpersist.variance [--shape c4|dense50] [--smoke] [--out FILE]
                                  [--motion-csv motion_trace_real.csv]

The analysis functions (`window_bytes`, `abba_orders`, `combo_stats`,
`policy_deltas`, `separated`) are plain Python for tests.
"""

from __future__ import annotations

import argparse
import csv
import glob
import hashlib
import json
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

SKIP, COUNT, REPEATS = 34, 16, 3
SPREAD_PASS = 0.10
HOT_RANGE = 0.20
MODES = ("dense", "stream")
POLICIES = ("none", "uniform", "recency", "motion", "reuse_weighted")
COMBOS = [(m, p) for m in MODES for p in POLICIES]
KERNEL = "attn_fwd_bf16_kernel"

# dtype, window (frames, 0 = full prefix), set-aside bytes, policies, the
# attention kernel and the split-combine kernel counted with it
SHAPES = {
    "c4": dict(dtype="bf16", window=8, set_aside=None, policies=POLICIES,
               kernel=KERNEL, follow="attn_combine_kernel",
               title="C4 (50 frames, window 8, bf16)"),
    "dense50": dict(dtype="fp32", window=0, set_aside=2162688,
                    policies=("none", "recency", "motion", "reuse_weighted"),
                    kernel="attn_fwd_f32_kernel", follow="attn_combine_kernel",
                    title="dense50 (50 frames, full causal prefix, fp32, 11-tile set-aside)"),
}

ROOT = Path(__file__).resolve().parents[2]


# ---------------------------------------------------------------- analysis --

def abba_orders(combos, repeats):
    """Run order per repeat: forward, reversed, forward, ... (reference :160)."""
    return [list(combos) if r % 2 == 0 else list(reversed(combos)) for r in range(repeats)]


def window_bytes(rows, skip=SKIP, count=COUNT, kernel=KERNEL, counter="FETCH_SIZE",
                 follow=None):
    """Per-launch counter values of the kernel's launches skip..skip+count-1.

    rows: dicts with Dispatch_Id, Kernel_Name, Counter_Name, Counter_Value
    (rocprofv3 counter_collection.csv). Launches are ordered by dispatch id.
    Dispatches of a `follow` kernel (the split combine) count toward the
    kernel launch dispatched before them.
    """
    per, extra = {}, {}
    for r in rows:
        if r["Counter_Name"] != counter:
            continue
        name = r["Kernel_Name"]
        d = int(r["Dispatch_Id"])
        if kernel in name:
            per[d] = per.get(d, 0.0) + float(r["Counter_Value"])
        elif follow and follow in name:
            extra[d] = extra.get(d, 0.0) + float(r["Counter_Value"])
    ids = sorted(per)
    if len(ids) < skip + count:
        raise ValueError(f"{counter}: {len(ids)} {kernel} launches, window needs {skip + count}")
    for d, val in extra.items():
        owner = [i for i in ids if i < d]
        if owner:
            per[owner[-1]] += val
    return [per[d] for d in ids[skip:skip + count]]


def combo_stats(sums, launches=None):
    """Median / min / max / spread of one combo's per-repeat sums, and the
    launches whose range across repeats exceeds 20 % of their median."""
    s = sorted(sums)
    n = len(s)
    med = s[n // 2] if n % 2 else 0.5 * (s[n // 2 - 1] + s[n // 2])
    spread = (s[-1] - s[0]) / med if med else 0.0
    hot = []
    if launches:
        for i in range(len(launches[0])):
            col = sorted(run[i] for run in launches)
            m = col[len(col) // 2] if len(col) % 2 else 0.5 * (col[len(col) // 2 - 1] + col[len(col) // 2])
            if m > 0 and (col[-1] - col[0]) / m > HOT_RANGE:
                hot.append(i)
    return {"median": med, "min": s[0], "max": s[-1], "spread": spread,
            "pass": spread <= SPREAD_PASS, "hot_launches": hot}


def overlap(a, b):
    """Do the [min, max] bands of two combo_stats overlap?"""
    return not (a["max"] < b["min"] or a["min"] > b["max"])


def policy_deltas(stats, mode):
    """Median delta of each gated policy vs none of the same mode, and whether
    its band overlaps none's."""
    base = stats[(mode, "none")]
    out = {}
    for p in POLICIES[1:]:
        s = stats.get((mode, p))
        if s:
            out[p] = {"delta": (s["median"] - base["median"]) / base["median"],
                      "overlaps_none": overlap(s, base)}
    return out


TRACE_ENV = "KVP_VARIANCE_MOTION_CSV"   # passes --motion-csv to the profiled children


def separated(stats, mode, a="reuse_weighted", b="recency"):
    return not overlap(stats[(mode, a)], stats[(mode, b)])


# ------------------------------------------------------------------ child --

def child(shape, mode, policy, out_json):
    """One run of the shape (one layer, 50 frames); writes the output digest."""
    sys.path.insert(0, str(ROOT / "cuda-kv-persistence_amd"))
    import torch
    from kvpersist import BF16, FP32, FramePipeline, workloads

    sh = SHAPES[shape]
    cfg = workloads.CONFIGS["c4"]
    T, D, H, F = cfg.tokens, workloads.HIDDEN, workloads.HEADS, cfg.frames
    fp32 = sh["dtype"] == "fp32"
    q, k, v = workloads.qkv_device(F, T, seed=42,
                                   dtype=torch.float32 if fp32 else torch.bfloat16,
                                   device="cuda")
    out = torch.empty_like(q)
    pl = FramePipeline(policy, cross=True, streaming=(mode == "stream"), frames=F, T=T, D=D,
                       heads=H, tile_tokens=workloads.TILE_TOKENS,
                       set_aside_bytes=sh["set_aside"] or cfg.set_aside,
                       dtype=FP32 if fp32 else BF16, window_frames=sh["window"])
    trace = os.environ.get(TRACE_ENV)
    if trace:
        from kvpersist.motion import read_trace_csv
        scores = read_trace_csv(trace)
        if scores.shape != (F, cfg.num_tiles):
            raise ValueError(f"{trace}: scores {scores.shape}, C4 needs ({F}, {cfg.num_tiles})")
    else:
        scores = workloads.motion_for(cfg, 0)
    pl.set_scores(scores)
    for f in range(F):
        pl.step(f, q, k, v, out)
    torch.cuda.synchronize()
    digest = hashlib.sha256(out.view(torch.int16 if not fp32 else torch.int32)
                            .cpu().numpy().tobytes()).hexdigest()
    pl.close()
    Path(out_json).write_text(json.dumps({"mode": mode, "policy": policy, "sha256": digest}))


# ----------------------------------------------------------------- parent --

def _profiled(counters, shape, mode, policy, workdir, tag, timeout):
    d = Path(workdir) / tag
    digest = Path(workdir) / f"{tag}.json"
    sh = SHAPES[shape]
    cmd = ["rocprofv3", "--pmc", *counters, "--kernel-include-regex",
           f"{sh['kernel']}|{sh['follow']}",
           "--output-format", "csv", "-d", str(d), "-o", "p", "--",
           sys.executable, "-m", "kvpersist.variance", "--shape", shape,
           "--child", mode, policy, str(digest)]
    env = dict(os.environ, TMPDIR=os.environ.get("TMPDIR", "/tmp"))
    env["PYTHONPATH"] = str(ROOT / "cuda-kv-persistence_amd") + os.pathsep + env.get("PYTHONPATH", "")
    # own process group: a run that overstays its limit is killed with the
    # program it profiles
    proc = subprocess.Popen(cmd, cwd=ROOT, env=env, stdout=subprocess.DEVNULL,
                            stderr=subprocess.DEVNULL, start_new_session=True)
    try:
        rc = proc.wait(timeout=timeout)
    except subprocess.TimeoutExpired:
        os.killpg(proc.pid, 9)
        proc.wait()
        raise RuntimeError(f"{tag}: rocprofv3 run exceeded {timeout} s")
    if rc != 0 or not digest.exists():
        raise RuntimeError(f"{tag}: rocprofv3 run failed (exit {rc})")
    rows = []
    for f in glob.glob(str(d / "**" / "*counter_collection.csv"), recursive=True):
        with open(f) as fh:
            rows.extend(csv.DictReader(fh))
    return rows, json.loads(digest.read_text())["sha256"]


def _fetch_factor():
    tj = ROOT / "profiles" / "attn_bf16_c3_traffic.json"
    try:
        return float(json.loads(tj.read_text())["calibration"]["fetch_factor"])
    except (OSError, KeyError, ValueError):
        return 1.0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shape", default="c4", choices=sorted(SHAPES))
    ap.add_argument("--child", nargs=3, metavar=("MODE", "POLICY", "OUT"))
    ap.add_argument("--smoke", action="store_true", help="one combo, one repeat")
    ap.add_argument("--out", default=None,
                    help="report path (default profiles/variance_<shape>.md)")
    ap.add_argument("--timeout", type=int, default=180, help="seconds per profiled run")
    ap.add_argument("--hit-repeats", type=int, default=REPEATS,
                    help="repeats that also run the L2 hit-rate pass")
    ap.add_argument("--motion-csv", default=None,
                    help="motion trace CSV (frame_id,tile_id,motion_score,...; 50 x 98 rows) "
                         "instead of the synthetic C4 scores, as the reference runs its "
                         "real-motion trace")
    args = ap.parse_args(argv)
    if args.motion_csv:
        os.environ[TRACE_ENV] = str(Path(args.motion_csv).resolve())
    if args.child:
        child(args.shape, *args.child)
        return 0
    if not shutil.which("rocprofv3"):
        print("rocprofv3 not found", file=sys.stderr)
        return 2
    sh = SHAPES[args.shape]
    out_path = args.out or str(ROOT / "profiles" / f"variance_{args.shape}.md")
    factor = _fetch_factor()
    shape_combos = [(m, p) for m in MODES for p in sh["policies"]]
    combos = shape_combos[:1] if args.smoke else shape_combos
    repeats = 1 if args.smoke else REPEATS
    results = {c: [] for c in combos}
    digests = {}
    with tempfile.TemporaryDirectory(prefix="kvp_var_") as work:
        for r, order in enumerate(abba_orders(combos, repeats)):
            for mode, policy in order:
                tag = f"{mode}_{policy}_r{r}"
                rows, dg = _profiled(["FETCH_SIZE"], args.shape, mode, policy, work,
                                     tag + "_fetch", args.timeout)
                fetch = [x * 1024.0 * factor
                         for x in window_bytes(rows, kernel=sh["kernel"], follow=sh["follow"])]
                rate = None
                if r < args.hit_repeats:
                    hrows, _ = _profiled(["TCC_HIT_sum", "TCC_MISS_sum"], args.shape, mode,
                                         policy, work, tag + "_hit", args.timeout)
                    hit = window_bytes(hrows, kernel=sh["kernel"], follow=sh["follow"],
                                       counter="TCC_HIT_sum")
                    miss = window_bytes(hrows, kernel=sh["kernel"], follow=sh["follow"],
                                        counter="TCC_MISS_sum")
                    rate = sum(hit) / max(1.0, sum(hit) + sum(miss))
                digests[(mode, policy, r)] = dg
                results[(mode, policy)].append({"launches": fetch, "sum": sum(fetch),
                                                "hit_rate": rate})
                print(f"[r{r}] {mode}/{policy}: window fabric reads {sum(fetch) / 1e9:.3f} GB"
                      + (f", L2 hit {100 * rate:.2f} %" if rate is not None else ""),
                      flush=True)
    gate = all(digests[(m, p, r)] == digests[(m, "none", r)]
               for (m, p, r) in digests if (m, "none", r) in digests)
    stats = {c: combo_stats([x["sum"] for x in results[c]], [x["launches"] for x in results[c]])
             for c in combos}
    md = [f"# Fabric-read variance and policy separation — {sh['title']}\n",
          f"Command (MI355X, repo root): `python3 -m kvpersist.variance --shape {args.shape}"
          + (f" --hit-repeats {args.hit_repeats}" if args.hit_repeats != REPEATS else "")
          + "` — per run a `rocprofv3 --pmc FETCH_SIZE` pass (and, in the first "
          f"{min(args.hit_repeats, repeats)} repeat(s), a `TCC_HIT_sum TCC_MISS_sum` pass) "
          f"restricted to `{sh['kernel']}` and `{sh['follow']}` (a frame's split combine "
          f"counted with its launch); window = frames {SKIP}..{SKIP + COUNT - 1} of 50; "
          f"{repeats} repeat(s), ABBA order; reads scaled x{factor:g} (copy calibration).\n",
          "Motion scores: " + (f"`{Path(args.motion_csv).name}` (`--motion-csv`)"
                               if args.motion_csv else
                               "the synthetic C4 field (`workloads.motion_for`)") + ".\n",
          f"Bitwise gate (every policy's output equals none's, same mode and repeat): "
          f"{'PASS' if gate else 'FAIL'}\n",
          "| mode | policy | window reads median | min | max | spread | L2 hit median | verdict |",
          "|---|---|---|---|---|---|---|---|"]
    all_pass = True
    for c in combos:
        s = stats[c]
        hits = sorted(x["hit_rate"] for x in results[c] if x["hit_rate"] is not None)
        all_pass &= s["pass"]
        md.append(f"| {c[0]} | {c[1]} | {s['median'] / 1e9:.4f} GB | {s['min'] / 1e9:.4f} | "
                  f"{s['max'] / 1e9:.4f} | {100 * s['spread']:.2f} % | "
                  + (f"{100 * hits[len(hits) // 2]:.2f} %" if hits else "n/a") + " | "
                  f"{'PASS' if s['pass'] else 'FAIL (excursion)'} |")
        if s["hot_launches"]:
            md.append(f"  - launches with > 20 % range: {len(s['hot_launches'])}/{COUNT} "
                      f"(window indices {s['hot_launches']})")
    if not args.smoke:
        md += ["\n## Policy deltas vs none (medians)\n",
               "| mode | policy | reads vs none | band overlaps none |", "|---|---|---|---|"]
        sep = {}
        for m in MODES:
            for p, d in policy_deltas(stats, m).items():
                md.append(f"| {m} | {p} | {100 * d['delta']:+.2f} % | "
                          f"{'yes' if d['overlaps_none'] else 'no'} |")
            sep[m] = separated(stats, m)
            md.append(f"  - [{m}] reuse_weighted vs recency bands: "
                      f"{'SEPARATED' if sep[m] else 'OVERLAP'}")
        verdict = ("VALIDATED" if all(sep.values()) else
                   "PARTIAL" if any(sep.values()) else "NOT_SUPPORTED")
        md += ["\n## Verdict\n",
               f"Measurement {'stable' if all_pass else 'UNSTABLE'} (every combo spread "
               f"<= {100 * SPREAD_PASS:.0f} %: {'yes' if all_pass else 'no'}); gating thesis "
               f"(reuse_weighted separated from recency in both modes): {verdict}."]
    text = "\n".join(md) + "\n"
    print(text)
    if not args.smoke:
        Path(out_path).write_text(text)
    return 0 if gate else 1


if __name__ == "__main__":
    sys.exit(main())
