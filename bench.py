"""AEISU 2x upscaling throughput on one MI355X (BASELINE.json metric).

Default workload = BASELINE config 2: 1920x1080 -> 3840x2160, batch 1, mixed
FP8-E4M3 / FP16 (weights/aeisu_area_mixed_fp8.bin), FP16 frames in and out.
A "step" is one frame through the whole path (controller + reconstruction
head).  Frames are seeded synthetic scenes (aeisu_amd.frames), a pool of
distinct frames resident in HBM before timing starts.

Protocol:
  0. --clock-warmup seconds (default 0.5) of untimed frames: the GPU reaches its
     sustained clocks only after milliseconds of load, longer than W frames take.
  1. W warm-up steps, then K timed steps of eager launches (the kernels of a
     frame on the current stream: two for the quantized policies, three for FP16), bracketed by torch.cuda.synchronize():
     value = K / elapsed (frames/s).  The same is measured for replays of the
     per-frame HIP graph and reported beside it (--graph makes that the value).
  1b. K steps processed synchronously, each between two HIP events on the launch
     stream (the reference's per-frame Process() timing): median and p95 per step.
  2. K more steps launched eagerly with HIP events recorded on the launch
     stream around every kernel: per-kernel average durations -> roofline.
  3. CPU baseline: the FP32 oracle restatement of the reference PyTorch path
     (oracle/model.py, tile=0) on a bounded sample of the same frames.

Prints ONE JSON line.  ``--table`` measures configurations 0-4 in one run (GPU and
CPU baseline each) and prints one line per configuration plus a markdown table.  ``--gpus N`` with N > 1 exits: this build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK = 8.0e12          # B/s, MI355X HBM3E
MFMA_PEAK = {"fp16": 2.5e15, "fp8": 5.0e15, "int8": 5.0e15, "fp32": 157.3e12}   # dense; fp32: MI355X FP32 peak
CTRL_MAC_FP16 = 256 + 4608 + 1024        # project + refine + tail, per LR pixel (paper tex:352-359)
CTRL_MAC_LOW = 512 + 4608 + 512          # compress + 4 bottlenecks + expand
WORKLOADS = {
    0: dict(precision="fp32", weights="aeisu_area.pt", name="aeisu_area fp32 256x256->512x512 b1"),
    1: dict(precision="fp16", weights="aeisu_area.pt", name="aeisu_area fp16 1080p->4K b1"),
    2: dict(precision="mixed", weights="aeisu_area_mixed_fp8.bin", name="aeisu_area mixed-fp8/fp16 1080p->4K b1"),
    3: dict(precision="int8", weights="aeisu_int8_fp16.pt", name="aeisu int8/fp16 540p->1080p b8"),
    4: dict(precision="mixed", weights="aeisu_div2k_l1_mixed_fp8.bin", name="aeisu_div2k_l1 mixed 1440p->5K b4"),
}


# the FP32 model whose reference PyTorch path the CPU baseline runs for each configuration (the INT8
# artifact of config 3 is quantized from aeisu_area.pt)
CPU_MODEL = {0: "aeisu_area.pt", 1: "aeisu_area.pt", 2: "aeisu_area.pt", 3: "aeisu_area.pt", 4: "aeisu_div2k_l1.pt"}


KERNEL_KEYS = {"project_kernel": "project", "body_fused_kernel": "body", "fused_tail_head_kernel": "refine_tail_head",
               "head_kernel": "head", "refine_tail_kernel": "refine_tail"}


PROFILE_TAGS = {1: "fp16_1080p", 2: "mixed_1080p", 3: "int8_540p_b8", 4: "mixed_1440p_b4"}


def measured_traffic(config: int):
    """HBM bytes per frame batch and stage from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE summary of
    the configuration (calibrated against 256 MiB device copies), keyed by stage."""
    path = ROOT / "profiles" / f"hbm_traffic_{PROFILE_TAGS.get(config, '')}_pmc.md"
    out = {}
    if path.exists():
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes "):
                _, name, value = line.split()
                out[KERNEL_KEYS.get(name, name)] = int(value)
    return out


def geometry(h, w):
    ey, ex = -h % 32, -w % 32
    return h + 32 + ey, w + 32 + ex


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_model() -> str:
    """CPU model name from /proc/cpuinfo (platform.processor() is empty on Linux)."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.machine()


def cpu_baseline(frames_cpu, budget_s: float, min_frames: int = 5, weights: str = "aeisu_area.pt"):
    """FP32 oracle (the reference PyTorch path restated) on whole frames: one warm-up frame, then at
    least ``min_frames`` timed frames, more while the budget lasts (BASELINE protocol: 1 + >= 5)."""
    import torch
    from oracle import model as M
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    threads = min(usable, int(os.environ.get("OMP_NUM_THREADS", usable)))
    torch.set_num_threads(threads)
    state = M.load_folded(ROOT / "weights" / weights)
    M.upscale(state, frames_cpu[0].float(), 0)             # warm-up: one whole frame
    done, t0 = 0, time.perf_counter()
    while done < min_frames or time.perf_counter() - t0 < budget_s:
        M.upscale(state, frames_cpu[done % len(frames_cpu)].float(), 0)
        done += 1
    elapsed = time.perf_counter() - t0
    return {"value": done / elapsed, "unit": "frames/s", "cores": threads, "kind": "port",
            "ms_per_frame": 1000 * elapsed / done, "cpu_model": cpu_model(), "threads": threads,
            "sample": f"1 warm-up + {done} timed whole {frames_cpu.shape[-2]}x{frames_cpu.shape[-1]} frames through "
                      f"oracle/model.py FP32 upscale(tile=0) of {weights} (torch CPU, {threads} threads on {usable} "
                      f"usable cores, {cpu_model()})"}


def median_p95(samples):
    """Median and 95th percentile of per-frame times as the reference's runtime test computes them
    (SrcPyrRuntimeTest.cpp:137-151 median, mean of the middle two for an even count; :240 p95 =
    sorted[min(n - 1, ceil(0.95 n) - 1)])."""
    import math
    v = sorted(samples)
    n = len(v)
    med = v[n // 2] if n % 2 else 0.5 * (v[n // 2 - 1] + v[n // 2])
    return med, v[min(n - 1, math.ceil(0.95 * n) - 1)]


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=2, choices=sorted(WORKLOADS))
    ap.add_argument("--pool", type=int, default=4, help="distinct resident frames cycled through")
    ap.add_argument("--cpu-budget", type=float, default=12.0, help="seconds of CPU-baseline work (0 = skip)")
    ap.add_argument("--graph", action="store_true",
                    help="report graph replays as the value (default: eager launches, which are faster here: "
                         "a graph launch costs more than the two or three kernel launches it replaces)")
    ap.add_argument("--unfused", action="store_true",
                    help="refine+tail and head as two kernels (coefficients through device memory)")
    ap.add_argument("--size", default=None, metavar="HxW",
                    help="input frame size override for resolution sweeps (the headline value is config 2)")
    ap.add_argument("--batch", type=int, default=None, help="batch override for sweeps")
    ap.add_argument("--precision", default=None,
                    help="precision policy override the weight file allows (fp16, fp32, mixed, mixed-fp8mma, int8)")
    ap.add_argument("--clock-warmup", type=float, default=0.5, metavar="S",
                    help="seconds of untimed frames before the warm-up steps, so the timed frames run at the "
                         "clocks a sustained load reaches")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of MIB MiB (reference point for HBM counters)")
    ap.add_argument("--table", action="store_true",
                    help="configurations 0-4 in one run, each on the GPU and on the CPU baseline (1 warm-up + "
                         ">= 5 frames): one JSON line per configuration, then a markdown table on stderr")
    return ap.parse_args()


def measure(args, config: int, size=None, batch=None, precision=None, cpu_budget: float = 0.0):
    """GPU (and optionally CPU-baseline) measurement of one configuration; returns the JSON record."""
    import torch
    from aeisu_amd import frames as FR
    from aeisu_amd import runtime as R
    from aeisu_amd import _lib as L

    wl = dict(WORKLOADS[config])
    spec = dict(FR.CONFIGS[config])
    if size:
        spec["height"], spec["width"] = size
    if batch:
        spec["batch"] = batch
    if precision:
        wl["precision"] = precision
    sweep = bool(size or batch or precision)
    B, H, W = spec["batch"], spec["height"], spec["width"]
    dev = torch.device("cuda", 0)
    log(f"bench: config {config} ({wl['name']}), generating {args.pool} frame batches")
    pool_cpu = [FR.config_frames(config, seed=1000 * i, batch=B, size=size) for i in range(args.pool)]
    pool = [p.to(dev).contiguous() for p in pool_cpu]
    io_dtype = pool[0].dtype                                   # FP16 frames (FP32 for config 0)
    outs = [torch.empty(B, 3, 2 * H, 2 * W, dtype=io_dtype, device=dev) for _ in pool]
    model = R.load_model(ROOT / "weights" / wl["weights"], precision=wl["precision"])
    stream = torch.cuda.current_stream()

    run_flags = L.FLAG_UNFUSED if args.unfused else 0

    def step(i, graph):
        j = i % len(pool)
        model.run(pool[j], out=outs[j], graph=graph, check_finite=False, flags=run_flags)

    # --- 1. timed region: eager launches (the frame's kernels) and graph replays ----------------
    def timed(graph):
        for i in range(args.warmup):
            step(i, graph)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            step(i, graph)
        torch.cuda.synchronize()
        return 1000 * (time.perf_counter() - t0) / args.steps

    model.run(pool[0], out=outs[0], flags=run_flags)         # finite check once, outside timing
    # The per-frame graphs are captured before the clock warm-up: capturing and instantiating them
    # leaves the GPU idle for long enough that it lowers its clocks, and the frames timed right after
    # ran up to 12 % slower (one box: 137.8 against 123.4 us per frame, recovering over about 60 frames).
    for j in range(len(pool)):
        step(j, True)
    torch.cuda.synchronize()
    # The GPU raises its clocks only after some milliseconds of load: W warm-up frames (~1 ms at
    # W = 5) leave the timed frames at a lower clock than a serving loop runs at (0.165-0.169 against
    # 0.143 ms per 1080p frame on one box).  Frames are run untimed for --clock-warmup seconds first.
    t_warm = time.perf_counter()
    n_warm = 0
    while time.perf_counter() - t_warm < args.clock_warmup:
        for _ in range(64):
            step(n_warm, False)
            n_warm += 1
        torch.cuda.synchronize()
    eager_launch_ms = timed(False)
    graph_ms = timed(True)
    graph = args.graph
    ms_per_step = graph_ms if graph else eager_launch_ms
    log(f"bench: {eager_launch_ms:.4f} ms/step eager, {graph_ms:.4f} ms/step graph replay "
        f"(value from {'graph' if graph else 'eager'})")

    # --- 1b. per-frame synchronous timing, the reference's Process() protocol ------------------------
    # SrcPyrRuntimeTest.cpp:195-240: every frame is processed synchronously and timed with device
    # events around it; the median and the 95th percentile over the frames are reported.  Here: HIP
    # events on the launch stream around each eager frame, the host waiting for each frame's end.
    per_frame = []
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for i in range(args.steps):
        ev0.record(stream)
        step(i, graph)
        ev1.record(stream)
        ev1.synchronize()
        per_frame.append(ev0.elapsed_time(ev1))
    frame_med, frame_p95 = median_p95(per_frame)
    log(f"bench: per-frame synchronous median {frame_med:.4f} ms, p95 {frame_p95:.4f} ms")

    # --- 2. per-kernel HIP events on the launch stream ---------------------------------------------
    hd = model.handle(B, H, W, io_dtype, io_dtype, L.FLAG_STAGE_TIMING | run_flags)
    for i in range(min(args.warmup, 5)):
        L.check(L.lib().aeisu_upscale_async(hd.ptr, pool[i % len(pool)].data_ptr(), outs[i % len(pool)].data_ptr(),
                                            stream.cuda_stream))
    model.stage_timings(hd, reset=True)
    t1 = time.perf_counter()
    for i in range(args.steps):
        j = i % len(pool)
        L.check(L.lib().aeisu_upscale_async(hd.ptr, pool[j].data_ptr(), outs[j].data_ptr(), stream.cuda_stream))
    torch.cuda.synchronize()
    eager_ms = 1000 * (time.perf_counter() - t1) / args.steps
    stages, nframes = model.stage_timings(hd, reset=True)
    log("bench: stage ms " + ", ".join(f"{k}={v:.4f}" for k, v in stages.items()))

    # --- algorithmic work per step -------------------------------------------------------------------
    Hp, Wp = geometry(H, W)
    lr_px = B * H * W
    packed_px = B * (Hp // 2) * (Wp // 2)
    s_io = pool[0].element_size()                             # frame bytes per value in and out
    head_bytes = lr_px * (3 * s_io + 16 * 2 + 12 * s_io)      # RGB in + FP16 coefficients + 2x RGB out
    refine_bytes = packed_px * (32 * 2 + 64 * 2)              # FP16 refine input + FP16 coefficient output
    refine_flops = 2.0 * packed_px * (32 * 64 * 9 + 64 * 64)
    synth_flops = 2.0 * lr_px * 16 * 100                      # head filter synthesis (MFMA)
    # MFMA the low-precision layers run on: the Mixed policy feeds E4M3 values to the FP16 MFMA
    # (exact products, FP32 accumulation), INT8 uses the i8 MFMA
    low_kind = {"fp16": "fp16", "mixed": "fp16", "mixed-fp8mma": "fp8", "int8": "int8", "fp32": "fp32"}[wl["precision"]]
    # the FP32 policy runs FP32 FMAs everywhere (per-layer kernels, no fused variants)
    hi_kind = "fp32" if wl["precision"] == "fp32" else "fp16"
    ctrl_flops16 = 2.0 * lr_px * CTRL_MAC_FP16
    ctrl_flops_low = 2.0 * lr_px * CTRL_MAC_LOW
    fused = not args.unfused and wl["precision"] != "fp32"   # fused body and fused refine+tail+head kernels
    traffic = {} if sweep else measured_traffic(config)       # the profiles cover configs 1-4 as defined
    kernels = {}
    proj_bytes = lr_px * 3 * s_io + packed_px * 32 * 2        # RGB in + FP16 skip out
    proj_flops = 2.0 * packed_px * 32 * 32                    # project 1x1, FP16 MFMA
    # the quantized policies' fused body computes analysis + project from the frames itself
    body_has_project = fused and stages["project"] == 0.0
    if not body_has_project:
        ps = stages["project"] / 1000
        kernels["project"] = {"bound": "hbm", "achieved": proj_bytes / ps / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                              "frac": proj_bytes / ps / HBM_PEAK, "ms": stages["project"],
                              "algorithmic_bytes": proj_bytes, "traffic": traffic.get("project")}
    if fused:
        # [project +] compress + 4 bottlenecks + expand in one kernel; in: RGB frames (or the FP16
        # skip tensor), out: FP16 work.  MFMA peak = the flop-weighted peak of the MFMAs it runs.
        bs_ = stages["bottleneck"] / 1000
        bflops = ctrl_flops_low + (proj_flops if body_has_project else 0.0)
        ideal_s = ctrl_flops_low / MFMA_PEAK[low_kind] + (proj_flops / MFMA_PEAK["fp16"] if body_has_project else 0.0)
        peak_eff = bflops / ideal_s
        body_bytes = (lr_px * 3 * s_io + packed_px * 32 * 2) if body_has_project else packed_px * 32 * 2 * 2
        kernels["body"] = {"bound": "mfma", "achieved": bflops / bs_ / 1e12,
                           "peak": peak_eff / 1e12, "unit": "TFLOP/s",
                           "frac": ideal_s / bs_, "ms": stages["bottleneck"],
                           "algorithmic_flops": bflops, "hbm_gbs": body_bytes / bs_ / 1e9,
                           "algorithmic_bytes": body_bytes, "traffic": traffic.get("body"),
                           "includes_project": body_has_project,
                           # SQ counters (profiles/sq_counters_*): VALU issue, not the MFMA, fills the SIMD
                           "limiter": "valu_issue"}
        if wl["precision"] == "mixed":
            # the reference quotes the Mixed arithmetic at the FP8 MFMA rate; this build runs its
            # E4M3 values on the FP16 MFMA (exact products, the reference's FP32 sums)
            fp8_ideal = ctrl_flops_low / MFMA_PEAK["fp8"] + (proj_flops / MFMA_PEAK["fp16"] if body_has_project else 0.0)
            kernels["body"]["frac_at_fp8_peak"] = fp8_ideal / bs_
        # work in + RGB in + 2x RGB out; coefficients never leave the chip
        fused_bytes = packed_px * 32 * 2 + lr_px * (3 * s_io + 12 * s_io)
        fs = stages["head"] / 1000
        kernels["refine_tail_head"] = {
            "bound": "hbm", "achieved": fused_bytes / fs / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
            "frac": fused_bytes / fs / HBM_PEAK, "ms": stages["head"], "algorithmic_bytes": fused_bytes,
            "traffic": traffic.get("refine_tail_head"),
            "mfma_tflops": (refine_flops + synth_flops) / fs / 1e12,
            "mfma_frac": (refine_flops + synth_flops) / fs / MFMA_PEAK["fp16"],
            "limiter": "valu_issue"}                          # HBM is priced; VALU issue fills the SIMD
        for k in ("compress", "expand", "refine_tail") + (("project",) if body_has_project else ()):
            stages.pop(k)                                     # empty on the fused path
        # controller = project + body + the refine/tail share of the fused kernel (by MFMA count)
        ctrl_ms = (stages.get("project", 0.0) + stages["bottleneck"]
                   + stages["head"] * refine_flops / (refine_flops + synth_flops))
    else:
        head_s = stages["head"] / 1000
        refine_s = stages["refine_tail"] / 1000
        kernels["head"] = {"bound": "hbm", "achieved": head_bytes / head_s / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                           "frac": head_bytes / head_s / HBM_PEAK, "ms": stages["head"],
                           "algorithmic_bytes": head_bytes, "traffic": traffic.get("head")}
        kernels["refine_tail"] = {"bound": "mfma" if hi_kind == "fp16" else "valu",
                                  "achieved": refine_flops / refine_s / 1e12,
                                  "peak": MFMA_PEAK[hi_kind] / 1e12, "unit": "TFLOP/s",
                                  "frac": refine_flops / refine_s / MFMA_PEAK[hi_kind], "ms": stages["refine_tail"],
                                  "algorithmic_flops": refine_flops, "traffic": traffic.get("refine_tail")}
        ctrl_ms = sum(stages[k] for k in ("project", "compress", "bottleneck", "expand", "refine_tail"))
    ctrl_ideal_s = ctrl_flops16 / MFMA_PEAK[hi_kind] + ctrl_flops_low / MFMA_PEAK[low_kind]
    dominant = max(kernels, key=lambda k: kernels[k]["ms"])
    roof = {k: v for k, v in kernels[dominant].items()
            if k in ("bound", "achieved", "peak", "unit", "frac", "traffic", "limiter")}
    roof["kernel"] = dominant

    if args.copy_calibration:
        # a plain copy kernel of known size: reads and writes exactly MIB MiB each
        n = args.copy_calibration * (1 << 20) // 4
        src_buf = torch.ones(n, dtype=torch.float32, device=dev)
        dst_buf = torch.empty_like(src_buf)
        for _ in range(3):
            dst_buf.copy_(src_buf)
        torch.cuda.synchronize()
        log(f"bench: copy calibration {args.copy_calibration} MiB x3 done")

    cpu = None
    if cpu_budget > 0:
        log("bench: CPU baseline")
        cpu = cpu_baseline(torch.cat(pool_cpu)[:2], cpu_budget, weights=CPU_MODEL[config])

    # the body's launch shape as configured (tile sides, halo exchange) from the startup report
    report = dict(kv.split("=", 1) for kv in hd.report().split() if "=" in kv)
    body_launch = {k: int(report[k]) for k in ("body_tiles24_frames", "body_tiles24_cols", "body_exchange_tile",
                                               "body_exchange_frames")
                   if k in report}

    fps = B * 1000.0 / ms_per_step
    return {
        "metric": "frames/s (ms/frame) 1080p->4K batch-1 mixed FP8/FP16; % MFMA / HBM roofline",
        "value": round(fps, 2), "unit": "frames/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5), "ms_per_frame": round(ms_per_step / B, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": {"fp16": "fp16", "mixed": "fp8-e4m3/fp16", "mixed-fp8mma": "fp8-e4m3/fp16",
                  "int8": "int8/fp16", "fp32": "fp32"}[wl["precision"]],
        "data": f"synthetic (aeisu_amd.frames config {config}, {args.pool} resident frames)",
        "config": {"workload": wl["name"] + (" (sweep override)" if sweep else ""), "config_id": config,
                   "batch": B, "input": [3, H, W],
                   "output": [3, 2 * H, 2 * W], "precision": wl["precision"], "weights": wl["weights"],
                   "io": str(io_dtype).replace("torch.", ""),
                   "timed": "graph replay" if graph else "eager launches",
                   "refine_tail_head": "two kernels" if args.unfused else "fused", "body_launch": body_launch},
        "roofline": roof,
        "cpu_baseline": cpu,
        "frame_ms": {"median": round(frame_med, 5), "p95": round(frame_p95, 5), "frames": len(per_frame),
                     "protocol": "synchronous per-step HIP events on the launch stream (reference Process())"},
        "kernels": kernels,
        "stages_ms": {k: round(v, 5) for k, v in stages.items()},
        "eager_ms_per_step": round(eager_launch_ms, 5), "graph_ms_per_step": round(graph_ms, 5),
        "eager_with_stage_events_ms_per_step": round(eager_ms, 5),
        "controller": {"ms": round(ctrl_ms, 5), "algorithmic_gflop": round((ctrl_flops16 + ctrl_flops_low) / 1e9, 3),
                       "mfma_frac": ctrl_ideal_s / (ctrl_ms / 1000), "ideal_ms_at_mfma_peak": ctrl_ideal_s * 1000,
                       "low_precision_mfma": low_kind},
        "timing_frames": nframes,
        "clock_warmup": {"seconds": args.clock_warmup, "frames": n_warm},
    }


def table_row(rec) -> str:
    """One row of the GPU/CPU comparison table (ms per frame, frames/s, cores, roofline fractions)."""
    b = rec["config"]["batch"]
    cpu = rec["cpu_baseline"] or {}
    head = rec["kernels"].get("refine_tail_head") or rec["kernels"].get("head")
    return (f"| {rec['config']['config_id']} | {rec['config']['workload']} | {cpu.get('ms_per_frame', 0):.1f} | "
            f"{cpu.get('value', 0):.2f} | {cpu.get('cores', '')} | {rec['ms_per_frame']:.4f} | {rec['value']:.0f} | "
            f"{rec['frame_ms']['median'] / b:.4f} / {rec['frame_ms']['p95'] / b:.4f} | "
            f"{100 * rec['controller']['mfma_frac']:.1f} | {100 * head['frac']:.1f} |")


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one MI355X; multi-GPU runs are out of scope "
              "(frames would shard across GPUs, one runtime per GPU, with no exchange)", file=sys.stderr)
        sys.exit(2)
    if args.table:
        rows = []
        for config in sorted(WORKLOADS):
            rec = measure(args, config, cpu_budget=max(args.cpu_budget, 1e-3))
            print(json.dumps(rec), flush=True)
            rows.append(table_row(rec))
        log("| config | workload | CPU ms/frame | CPU frames/s | cores | GPU ms/frame | GPU frames/s | "
            "GPU per-frame median / p95 ms | controller % MFMA peak | head % HBM peak |")
        log("|---|---|---|---|---|---|---|---|---|---|")
        for r in rows:
            log(r)
        return
    size = tuple(int(v) for v in args.size.lower().split("x")) if args.size else None
    rec = measure(args, args.config, size=size, batch=args.batch, precision=args.precision,
                  cpu_budget=args.cpu_budget)
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
