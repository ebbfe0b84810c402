#!/usr/bin/env python3
"""Headline benchmark: ms per forward+backward and Mpix/s of the batched
rasterizer at 4096x4096, 65,536 splats, B=1 on one MI355X.

A step is one call of rasterize_projected_gaussians on GPU-resident inputs
followed by backward with loss = sum(image * w) (w fixed, seeded), i.e. the
whole public-API path: depth sort, binning, pair sort, forward compositing,
backward compositing, gradients in the original order.  Before the warmup
steps, untimed steps run for --clock-ramp seconds (0.25) so that the timed
steps run at the GPU's working clocks (reported as `clock_ramp`).

Prints ONE JSON line.  `roofline` is for the dominant kernel (the backward
compositor, which dominates step time): its launch time is measured live with
HIP events (torch.cuda.Event on the stream the library launches on) over the
timed steps.  `stage_ms` / `stage_roofline` give every kernel of the step, timed
by events attached to each launch over a few untimed steps after the timed
region (the same path; gsplat_hip_trace_launches).  `cpu_baseline` times the CPU oracle (the C
restatement of the reference algorithm, oracle/tile_oracle.c, on the host's
threads) on the same scene, forward+backward, once, and the reference's
dense Torch renderer on config 0.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--config 2] [--clock-ramp 0.25]
    python bench.py --trace FILE --height H --width W [--trace-batch B] [--trace-gaussians G]
        a recorded scene (torch.save dict of means2d/conics/colors/opacities/depths,
        the reference's real-trace format) instead of a synthetic config

Measurement helpers (used for the committed rocprofv3 summaries):
    python bench.py --calibrate-copy     a plain copy of 256 MiB (read + write),
                                         run under rocprofv3 --pmc FETCH_SIZE /
                                         WRITE_SIZE to convert those counters
                                         into bytes
    python bench.py --summarize DIR      markdown summary of the rocprofv3 CSV
                                         output in DIR (kernel stats and/or
                                         counter collection)
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "fast-mac-gsplat_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

KEYS = ("means2d", "conics", "colors", "opacities", "depths")
PEAK_FP32_TFLOPS = 157.3   # MI355X published fp32 peak
PEAK_HBM_GBS = 8000.0      # MI355X published HBM3E bandwidth


# Algorithmic work of one launch of each kernel the step runs, from the
# per-unit figures of the measurement plan: (bound, bytes or FLOP, what is
# counted), in BG splats, N tile pairs, T tiles and `walked` pairs (each tile's
# list up to its stop).  Bytes are those a kernel must move (reads + writes);
# FLOP for the compositors are per (pixel, walked pair) evaluation.
def kernel_work(name, BG, N, walked, T):
    table = {
        "count_depth_runs_kernel": ("hbm", 40.0 * BG,
                                    "40 B/splat: count 24 read + 4 written, depth runs 4 read + 8 written"),
        "rank_pack_kernel": ("hbm", 120.0 * BG, "120 B/splat: run keys+values 8, attributes 36, count 4 read; "
                                                "record 64, perm 4, count 4 written"),
        "emit_kernel<true>": ("hbm", 32.0 * BG + 8.0 * N, "32 B/splat (record 24, count 4 read, offset 4 written) "
                                                         "+ 8 B/pair (key, value)"),
        "emit_kernel<false>": ("hbm", 28.0 * BG + (5.0 if N >= 1 << 23 else 8.0) * N,
                               "28 B/splat (record 24, offset 4) + 8 B/pair (key, value), or 5 B/pair (packed word "
                               "+ low tile byte) for the two-pass sort of 2^23+ pairs"),
        "emit_kernel<orig>": ("hbm", 44.0 * BG + (5.0 if N >= 1 << 23 else 8.0) * N + N / 8.0,
                              "44 B/splat (the count's record 36, offset + gid 8) + 5 or 8 B/pair as "
                              "emit_kernel<false> + the count's hit ballots (1 bit per candidate, at least one "
                              "per pair)"),
        "count_kernel": ("hbm", 104.0 * BG + N / 8.0, "104 B/splat (one-call path): means 8, conic 12, opacity 4, "
                                                      "colours 12 read, count 4 and the 64-B record written; "
                                                      "+ the hit ballots (1 bit per candidate, at least one per pair)"),
        "depth_run_sort_kernel": ("hbm", 12.0 * BG, "12 B/splat: depth 4 read, run key + value 8 written"),
        "depth_run_rank_kernel": ("hbm", 12.0 * BG, "12 B/splat: run key + value 8 read, perm 4 written"),
        "pack_kernel": ("hbm", 144.0 * BG, "144 B/splat: perm 4 and the count's 64-B record read; record 64, "
                                           "offset 4 and the original-order offset + gid 8 written (one-call path)"),
        "rs_global_hist_kernel(depth)": ("hbm", 4.0 * BG, "4 B/splat (depth keys read)"),
        "rs_global_hist_kernel(keys)": ("hbm", 4.0 * N, "4 B/pair (keys read)"),
        "rs_onesweep_kernel(depth)": ("hbm", 16.0 * BG, "16 B/splat per pass (key + value read and written)"),
        "rs_onesweep_kernel(keys)": ("hbm", 16.0 * N, "16 B/pair per pass (key + value read and written)"),
        "ranges_kernel": ("hbm", 4.0 * N + 4.0 * T, "4 B/pair (sorted keys read) + 4 B/tile (offsets written)"),
        "rs_block_counts_kernel(pairs:lo)": ("hbm", 1.0 * N + 1024.0 * -(-N // 8192),
                                             "1 B/pair (low tile bytes read) + 1 KB per 8192-pair block (counts "
                                             "written)"),
        "rs_block_scan_kernel(pairs:lo)": ("hbm", 2048.0 * -(-N // 8192),
                                           "2 KB per 8192-pair block (counts read, prefixes written)"),
        "rs_onesweep_kernel(pairs:lo)": ("hbm", 9.0 * N, "9 B/pair: low tile byte + packed word read, word written"),
        "rs_onesweep_kernel(pairs:hi)": ("hbm", 8.0 * N + 4.0 * T, "8 B/pair: word read, gid written; 4 B/tile"),
        "ranges_finish_kernel": ("hbm", 8.0 * T + 64.0 * BG, "8 B/tile (offsets read) + 64 B/splat (gradient "
                                                            "records zeroed)"),
        "bucket_sort_kernel": ("hbm", 12.0 * N + 4.0 * T + 64.0 * BG,
                               "12 B/pair (key, value read; id written) + 4 B/tile + 64 B/splat (gradient record "
                               "zeroed)"),
        "render_grads_unpack_kernel": ("hbm", 164.0 * BG, "164 B/splat: record 64 read, gradients 36 written, "
                                                          "record 64 zeroed"),
        "project_fwd_kernel": ("hbm", 72.0 * BG, "72 B/splat: 44 read + 28 written"),
        "project_bwd_kernel": ("hbm", 116.0 * BG, "116 B/splat: 72 read + 44 written"),
        "render_fwd_kernel": ("valu", 256.0 * walked * FLOP_PER_EVAL["render_forward"],
                              "256 x walked pairs x 24 FLOP"),
        "render_bwd_kernel": ("valu", 256.0 * walked * FLOP_PER_EVAL["render_backward"],
                              "256 x walked pairs x 60 FLOP"),
    }
    return table.get(name)


def stage_roofline(stage_ms, BG, N, walked, T):
    """Achieved fraction of each kernel's roof: its algorithmic work per launch (kernel_work) over
    its mean traced launch time."""
    out = {}
    for name, ms in stage_ms.items():
        w = kernel_work(name, BG, N, walked, T)
        if w is None or ms <= 0:
            continue
        bound, units, what = w
        if bound == "hbm":
            a = units / (ms * 1e-3) / 1e9
            out[name] = {"bound": "hbm", "achieved": round(a, 1), "unit": "GB/s", "frac": round(a / PEAK_HBM_GBS, 4),
                         "work": what}
        else:
            a = units / (ms * 1e-3) / 1e12
            out[name] = {"bound": "valu", "achieved": round(a, 2), "unit": "TFLOP/s",
                         "frac": round(a / PEAK_FP32_TFLOPS, 4), "work": what}
    return out


# The reference's best published cfg2 forward+backward: 65.754 ms on an Apple
# M4 (v8_direct; benchmarks/full_rasterizer_benchmark_v8_prior_compare_4k64k.md:34)
# = 4096*4096 / 65.754 ms = 255.15 Mpix/s.
REFERENCE_MPIX_S = {2: 4096 * 4096 / 65.754e-3 / 1e6}
# Algorithmic work per unit (per (pixel, tile-pair) evaluation inside a tile's
# processed range, upper bound 256 per pair): forward ~24 FLOP, backward ~60.
FLOP_PER_EVAL = {"render_forward": 24.0, "render_backward": 60.0}
# The dominant call's duration is sampled on every TIMED_SAMPLE-th timed step.
TIMED_SAMPLE = 4
# Untimed steps for this long come before the warmup steps.  The GPU raises
# its clocks over the first ~20-30 ms of continuous work, and an idle of
# ~50 ms lowers them again: after 5 warmup steps the next 20 cfg2 steps took
# 334 us on average and steps 50-300 took 295 us; after 200 steps of
# continuous work the next 20 took 292 us.  Without the ramp a short timed
# region (20 steps of 0.3 ms) would measure the clock transition, not the
# step.
CLOCK_RAMP_S = 0.25


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _host_threads() -> int:
    """Threads the CPU legs use: OMP_NUM_THREADS (the box's CPU share) or the core count."""
    raw = os.environ.get("OMP_NUM_THREADS", "")
    return int(raw) if raw.isdigit() and int(raw) > 0 else (os.cpu_count() or 1)


def cpu_baseline(sc, H, W, B, G, w_np):
    """The CPU baselines, timed on this host (reported beside the GPU figure,
    not the optimisation target):
      * value: the C restatement of the reference's tile algorithm
        (oracle/tile_oracle.c, OpenMP over tiles and splats) on the full
        workload, one forward + backward (binning, compositing, gradients);
      * dense_torch_cfg0: the reference's dense Torch renderer torch_direct
        (benchmarks/benchmark_full_matrix.py:128-152, restated in
        oracle/dense_reference.py, no early stop) on config 0 (512x512,
        512 splats), forward + loss.backward(), with torch's CPU threads set
        to the same count; median of 3 after one warm-up.  The dense
        renderer's autograd graph does not fit in memory at configs 1-4."""
    import numpy as np
    import torch

    from oracle import tile_oracle as TO
    from oracle.dense_reference import dense_reference
    from torch_gsplat_bridge_fast.scenes import make_scene_2d

    n = _host_threads()
    TO.set_threads(n)
    meta = TO.make_meta(H, W, B, G)
    s = TO.Scene(*(sc[k].numpy() for k in KEYS), B, G)
    t0 = time.perf_counter()
    bins = TO.bin_scene(meta, s)
    TO.render_forward(meta, s, bins)
    TO.render_backward(meta, s, bins, w_np)
    dt = time.perf_counter() - t0

    torch.set_num_threads(n)
    sc0 = make_scene_2d(0, seed=0)
    H0, W0 = sc0["H"], sc0["W"]
    w0 = torch.rand(H0, W0, 3, generator=torch.Generator().manual_seed(123))
    times = []
    for _ in range(4):
        ts = [sc0[k][0].clone().requires_grad_(k != "depths") for k in KEYS]
        t1 = time.perf_counter()
        img = dense_reference(*ts, H0, W0, early_stop=False)
        (img * w0).sum().backward()
        times.append(time.perf_counter() - t1)
    dense_s = float(np.median(times[1:]))
    return {
        "value": (B * H * W) / dt / 1e6,
        "unit": "Mpix/s",
        "ms_per_step": dt * 1e3,
        "cores": n,
        "kind": "port",
        "sample": f"full workload ({W}x{H}, B={B}, G={G}), one forward+backward of the C restatement of the "
                  f"reference tile algorithm on {n} threads (OpenMP); CPU: {_cpu_model()}, "
                  f"{os.cpu_count()} logical CPUs visible",
        "dense_torch_cfg0": {
            "value": H0 * W0 / dense_s / 1e6,
            "unit": "Mpix/s",
            "ms_per_step": dense_s * 1e3,
            "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": "config 0 (512x512, 512 splats): the reference's dense torch_direct renderer restated "
                      "(oracle/dense_reference.py, no early stop), fp32 forward + loss.backward(), median of 3",
        },
    }


CALIBRATION_BYTES = 256 << 20


def calibrate_copy() -> int:
    """One elementwise copy kernel (dst = src * 1) over CALIBRATION_BYTES, three
    times: under rocprofv3 --pmc its FETCH_SIZE / WRITE_SIZE per dispatch,
    divided by the bytes really moved, is the counter-to-bytes factor."""
    import torch

    dev = torch.device("cuda:0")
    src = torch.ones(CALIBRATION_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "kernel": "at::native elementwise mul (dst = src * 1)",
                      "bytes_read": CALIBRATION_BYTES, "bytes_written": CALIBRATION_BYTES, "dispatches": 3}))
    return 0


def summarize(d: str) -> int:
    """Markdown tables from rocprofv3 --output-format csv results under d."""
    import csv
    import glob
    from collections import defaultdict

    for path in sorted(glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)):
        rows = list(csv.DictReader(open(path)))
        total = sum(float(r["TotalDurationNs"]) for r in rows) or 1.0
        print(f"kernel stats: {os.path.relpath(path, d)}\n")
        print("| kernel | calls | avg us | min us | max us | share |")
        print("|---|---:|---:|---:|---:|---:|")
        for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
            print(f"| `{r['Name'][:90]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                  f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                  f"{100.0 * float(r['TotalDurationNs']) / total:.1f}% |")
        print()
    for path in sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)):
        acc = defaultdict(lambda: defaultdict(list))
        for r in csv.DictReader(open(path)):
            name = r.get("Kernel_Name", "")
            key = (r.get("Dispatch_Id", ""), r.get("Counter_Name", ""))
            acc[name][key].append(float(r.get("Counter_Value", "0") or 0.0))
        print(f"counters (mean per dispatch, summed over hardware instances): {os.path.relpath(path, d)}\n")
        print("| kernel | counter | dispatches | mean per dispatch |")
        print("|---|---|---:|---:|")
        for name, per in sorted(acc.items()):
            by_counter = defaultdict(list)
            for (disp, cname), vals in per.items():
                by_counter[cname].append(sum(vals))
            for cname, vals in sorted(by_counter.items()):
                print(f"| `{name[:70]}` | {cname} | {len(vals)} | {sum(vals) / len(vals):.6g} |")
        print()
    return 0


def main() -> int:
    if "--summarize" in sys.argv:
        return summarize(sys.argv[sys.argv.index("--summarize") + 1])
    if "--calibrate-copy" in sys.argv:
        return calibrate_copy()
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--clock-ramp", type=float, default=CLOCK_RAMP_S,
                    help="seconds of untimed steps before the warmup (0: none)")
    ap.add_argument("--config", type=int, default=2, help="scene config id (torch_gsplat_bridge_fast.scenes)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--trace", default="", help="recorded scene file (real-trace case)")
    ap.add_argument("--height", type=int, default=0, help="image height for --trace")
    ap.add_argument("--width", type=int, default=0, help="image width for --trace")
    ap.add_argument("--trace-batch", type=int, default=0, help="keep the first B images of the trace")
    ap.add_argument("--trace-gaussians", type=int, default=0, help="keep the first G splats per image")
    args = ap.parse_args()
    if args.trace and (args.height <= 0 or args.width <= 0):
        print("--trace needs --height and --width", file=sys.stderr)
        return 2

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: every box in this build has one MI355X and the path has no "
              f"cross-GPU step (got --gpus {args.gpus}, WORLD_SIZE {world}); run with --gpus 1.", file=sys.stderr)
        return 2

    import numpy as np
    import torch

    from torch_gsplat_bridge_fast import (RasterConfig, _ops, project_pinhole_gaussians,
                                          rasterize_pinhole_gaussians, rasterize_projected_gaussians)
    from torch_gsplat_bridge_fast.rasterize import _meta as raster_meta
    from torch_gsplat_bridge_fast.scenes import CONFIGS, load_trace, make_scene_2d, make_scene_3d

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    three_d = not args.trace and CONFIGS[args.config]["kind"] == "3d"
    if args.trace:
        sc = load_trace(args.trace, batch=args.trace_batch, gaussians=args.trace_gaussians)
        sc.update(H=args.height, W=args.width, B=sc["means2d"].shape[0], G=sc["means2d"].shape[1])
        leaves = [sc[k].to(dev).requires_grad_(k != "depths") for k in KEYS]
        workload = f"real_trace:{os.path.basename(args.trace)}"
    elif three_d:
        # Config 4: projection + rasterization, gradients to means3d/scales/quats/opacities.
        sc = make_scene_3d(seed=0)
        keys3 = ("means3d", "scales", "quats", "opacities")
        leaves = [sc[k].to(dev).requires_grad_(True) for k in keys3]
        colors3 = sc["colors"].to(dev)
        c2w = sc["camera_to_world"].to(dev)
        cam = (sc["fx"], sc["fy"], sc["cx"], sc["cy"])
    else:
        sc = make_scene_2d(args.config, seed=0)
        leaves = [sc[k].to(dev).requires_grad_(k != "depths") for k in KEYS]
    if not args.trace:
        workload = CONFIGS[args.config]["name"]
    H, W, B, G = sc["H"], sc["W"], sc["B"], sc["G"]
    w_cpu = torch.rand(B, H, W, 3, generator=torch.Generator().manual_seed(123))
    w = w_cpu.to(dev)
    cfg = RasterConfig(height=H, width=W)

    def op_means(events):
        per_op = {}
        for name, e0, e1 in events:
            per_op.setdefault(name, []).append(e0.elapsed_time(e1))
        return {k: float(np.mean(v)) for k, v in per_op.items()}

    def step():
        for t in leaves:
            t.grad = None
        if three_d:
            img = rasterize_pinhole_gaussians(*leaves, colors3, *cam, camera_to_world=c2w, config=cfg)
        else:
            img = rasterize_projected_gaussians(*leaves, cfg)
        img.backward(w)

    # Clock ramp (untimed, uninstrumented): one step, whose launches may
    # still load kernels, then continuous steps for args.clock_ramp seconds.
    ramp_steps = 0
    ramp_s = 0.0
    if args.clock_ramp > 0:
        step()
        ramp_steps = 1
        r0 = time.perf_counter()
        while time.perf_counter() - r0 < args.clock_ramp:
            step()
            ramp_steps += 1
        ramp_s = time.perf_counter() - r0

    # Warm-up (untimed), with the compositor calls bracketed to find the
    # dominant one.
    compositors = ("render_forward", "render_backward")
    _ops.set_timing(True, ops=compositors, pool=4 * max(args.warmup, 1))
    for _ in range(max(args.warmup, 1)):
        step()
    torch.cuda.synchronize()
    warm_ms = op_means(_ops.pop_timing())
    dom = max(compositors, key=lambda k: warm_ms.get(k, 0.0))

    # Timed region: wall clock over exactly `steps` steps.  Inside it the
    # dominant compositor of every 4th step is timed by HIP events (created
    # up front) that its kernel launch records (the kernel's own duration)
    # for the roofline figure; the other calls and steps are not
    # instrumented, since a launch with events costs the stream ~12 us.
    _ops.set_timing(True, ops=(dom,), pool=2 * args.steps, every=min(TIMED_SAMPLE, max(args.steps, 1)))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    comp_ms = op_means(_ops.pop_timing())
    ms_per_step = (t1 - t0) * 1e3 / args.steps

    # Per-kernel breakdown, after the timed region: every kernel launch of
    # n_stage untimed steps of the same path carries HIP events attached to
    # the launch itself (gsplat_hip_trace_launches), so each figure is that
    # kernel's own duration in the step's own launch sequence.
    n_stage = max(1, min(args.steps, 5))
    trace = _ops.LaunchTrace(capacity=min(1024, 64 * n_stage))
    with trace:
        for _ in range(n_stage):
            step()
    per_kernel = {}
    for name, ms in trace.launches:
        per_kernel.setdefault(name, []).append(ms)
    stage_ms = {k: float(np.mean(v)) for k, v in per_kernel.items()}
    stage_launches = {k: len(v) / n_stage for k, v in per_kernel.items()}

    with torch.no_grad():
        if three_d:
            m2, cq, op, dp = project_pinhole_gaussians(*leaves, *cam, camera_to_world=c2w)
            flat = (m2, cq, colors3, op, dp)
        else:
            flat = leaves
        meta = raster_meta(cfg, B, G)
        st = _ops.bin_gaussians(meta, *(t.detach().reshape(B * G, -1).squeeze(-1).contiguous() for t in flat))
        # pairs up to each tile's stop: the pairs a compositor must evaluate
        # (equal to N unless pixels saturate before a tile's list ends)
        walked = int(_ops.render_forward(meta, st, save_state=True)[3].sum().item())
    n_pairs = st.n_pairs
    n_tiles = B * ((H + 15) // 16) * ((W + 15) // 16)
    evals = 256.0 * walked
    achieved_tflops = evals * FLOP_PER_EVAL[dom] / (comp_ms[dom] * 1e-3) / 1e12
    traffic = None
    tpath = os.path.join(ROOT, "profiles", f"traffic_{dom}_cfg{args.config}.json")
    if not args.trace and os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    mpix = B * H * W / (ms_per_step * 1e-3) / 1e6
    line = {
        "metric": "ms per fwd+bwd (and Mpix/s) at 4096² / 64K splats B=1 on 1 MI355X",
        "value": round(mpix, 2),
        "unit": "Mpix/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_ramp": {"steps": ramp_steps, "seconds": round(ramp_s, 3)},
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": (round(mpix / REFERENCE_MPIX_S[args.config], 2)
                        if args.config in REFERENCE_MPIX_S and not args.trace else None),
        "dtype": "f32",
        "data": ("recorded trace (resident in HBM)" if args.trace else
                 "synthetic (seeded BASELINE config scene, generated on CPU, resident in HBM)"),
        "config": {
            "workload": workload,
            "height": H, "width": W, "batch": B, "gaussians": G,
            "tile_pairs": n_pairs,
            "walked_pairs": walked,
            "loss": "sum(image * w), w ~ U(0,1) seed 123",
            "parallelism": "single GPU",
        },
        "stage_source": f"kernel trace of {n_stage} untimed steps after the timed region (events attached to "
                        "each launch, gsplat_hip_trace_launches): mean ms per launch, launches per step",
        "stage_ms": {k: round(v, 4) for k, v in sorted(stage_ms.items(), key=lambda kv: -kv[1])},
        "stage_launches_per_step": stage_launches,
        "stage_roofline": stage_roofline(stage_ms, B * G, n_pairs, walked, n_tiles),
        "roofline": {
            "kernel": f"{dom} ({'render_bwd_kernel' if dom == 'render_backward' else 'render_fwd_kernel'})",
            "launch_us": round(comp_ms[dom] * 1e3, 2),
            "bound": "valu",
            "achieved": round(achieved_tflops, 3),
            "peak": PEAK_FP32_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved_tflops / PEAK_FP32_TFLOPS, 4),
            "traffic": traffic,
            "work": f"256 * walked_pairs evaluations x {FLOP_PER_EVAL[dom]:.0f} FLOP per launch",
            # the same launch against the HBM roof (measured bytes per launch
            # over the live launch time): shows the kernel is not HBM bound
            "hbm_achieved_gbs": (round(traffic / (comp_ms[dom] * 1e-3) / 1e9, 1) if traffic else None),
            "hbm_frac": (round(traffic / (comp_ms[dom] * 1e-3) / 1e9 / PEAK_HBM_GBS, 4) if traffic else None),
        },
    }
    if not args.no_cpu_baseline and not three_d:
        line["cpu_baseline"] = cpu_baseline({k: sc[k] for k in KEYS}, H, W, B, G, w_cpu.numpy())
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
