"""Benchmark: trained bytes/s of Leo's per-byte training step on one MI355X.

One benchmark step is one logical batch of the workload (L stories, one device
lane each) through the whole training path: the lane-parallel story pass, the
batch-end lane-ordered mean, and 30% bounded-surprise replay on the canonical
runtime -- the reference benchmark's input_bytes_per_second definition
(crates/leo-cli/src/main.rs:716,768: story bytes / wall seconds including
replay and merge). Synthetic seeded stories and a seeded synthetic model of the
workload's shape; nothing is skipped inside the timed region.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload D] [--no-replay]

The default workload is D (1,048,576 units, fan-in 64,
64 story lanes, 30% replay), the configuration the headline metric is quoted
on. Prints one JSON line. The roofline object prices the step kernel's work
counters with the per-lane-step byte model of leo_runtime.hip (step_bytes) and
divides by the summed HIP-event time of its launches inside the timed region;
roofline.sections splits the same figures into the story pass (story lanes),
the replay (canonical runtime) and the batch-end mean (merge kernel).
cpu_baseline times the CPU oracle (this repository's restatement of Leo's CPU
executor, one thread per story as in training.rs:1669-1683) on a bounded sample
of one batch of the same workload.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0


_HIP = None


def _device_sync() -> None:
    global _HIP
    if _HIP is None:
        _HIP = ctypes.CDLL("libamdhip64.so")
    if _HIP.hipDeviceSynchronize() != 0:
        raise RuntimeError("hipDeviceSynchronize failed")


# Bounded CPU sample: at a million units the oracle trains ~12 bytes/s per
# thread (with replay), so large workloads time the first min(lanes, cores)
# stories of the batch truncated to a prefix (about half a minute of CPU work).
CPU_PREFIX = {"D": 128, "E": 64}
# host threads a GPU box grants one GPU's job, whatever the machine reports
HOST_SHARE = 16


def host_cpu():
    """(cores this process may use, capped at the box's per-GPU share; nproc; CPU model)."""
    nproc = os.cpu_count() or 1
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = nproc
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return min(usable, HOST_SHARE), nproc, model


def cpu_baseline(workload, model, data, offsets, replay: bool):
    """Time the CPU oracle on one batch of the same workload (bounded sample):
    one thread per story as training.rs:1669-1683 runs them, min(lanes, cores)
    stories."""
    from oracle import binding

    cores, nproc, cpu_model = host_cpu()
    stories = [data[int(offsets[i]):int(offsets[i + 1])].tobytes() for i in range(len(offsets) - 1)]
    sample = "1 batch"
    if workload.name in CPU_PREFIX:
        count, prefix = min(len(stories), cores), CPU_PREFIX[workload.name]
        stories = [s[:prefix] for s in stories[:count]]
        sample = f"the batch's first {count} stories truncated to {prefix} bytes"
    rt = binding.OracleRuntime(model)
    started = time.perf_counter()
    rt.train_story_batch(stories, binding.TRAINING, replay=replay)
    seconds = time.perf_counter() - started
    nbytes = sum(len(s) for s in stories)
    return {
        "value": nbytes / seconds,
        "unit": "bytes/s",
        "cores": min(len(stories), cores),
        "nproc": nproc,
        "cpu_model": cpu_model,
        "kind": "port",
        "sample": f"{sample} of workload {workload.name}: {len(stories)} stories, {nbytes} bytes, "
                  f"replay {'on' if replay else 'off'}, {seconds:.1f} s",
    }


def copy_calibration(mib: int = 256, repeats: int = 4) -> int:
    """Plain device copy of a known size, for scaling the FETCH_SIZE/WRITE_SIZE
    counters of a profiled run into HBM bytes (torch's elementwise copy kernel)."""
    import torch

    n = mib * (1 << 20) // 4
    src = torch.arange(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(repeats):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes_per_dispatch": n * 4, "dispatches": repeats}), flush=True)
    return 0


def measured_traffic(workload: str):
    """HBM bytes per step-kernel launch from the committed PMC summary of this
    workload (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by the copy-kernel
    calibration), or None when no summary exists."""
    path = ROOT / "profiles" / f"leo_lane_steps_workload{workload}_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def canonical_steps(workload: str, frozen: int, supervised: int) -> int:
    """Per-step kernel time of the canonical runtime, the lane that runs the
    serial replay: `frozen` FROZEN steps of one document (a replay prefix,
    advance_frozen_batch, backend.rs:428-431) and `supervised` TRAINING steps
    (replay targets, training_step_batch, backend.rs:413-422), timed with HIP
    events over the step-kernel launches. With LEO_HIP_PHASE_PROFILE=1 the line
    also carries the per-phase work and barrier-wait time of one workgroup of
    the lane (LEO_HIP_PROFILE_PART picks which) in microseconds per step."""
    from leo_amd import native
    from leo_amd.runtime import HipRuntime
    from leo_amd.workload import WORKLOADS, synthetic_stories, workload_model

    w = WORKLOADS[workload]
    model = workload_model(w)
    data, offsets = synthetic_stories(w, 64)
    text = bytes(data)
    need = max(frozen, supervised) + 201
    while len(text) < need:
        text += text
    runtime = HipRuntime(model, device=0, max_lanes=1)
    profiled = os.environ.get("LEO_HIP_PHASE_PROFILE", "0") not in ("", "0")

    def timed(label, run, steps):
        runtime.kernel_stats(reset=True)
        started = time.perf_counter()
        run()
        wall = time.perf_counter() - started
        ks = runtime.kernel_stats()
        out = {"metric": f"canonical {label} step", "workload": w.name, "steps": steps,
               "kernel_us_per_step": ks["kernel_ms"] * 1e3 / steps, "wall_us_per_step": wall * 1e6 / steps,
               "launches": ks["launches"], "active_per_step": ks["active"] / steps,
               "events_per_step": ks["events"] / steps, "touched_per_step": ks["touched"] / steps}
        if profiled:
            out["phase_work_us"] = [round(x / steps, 3) for x in ks["phase_work_us"]]
            out["phase_wait_us"] = [round(x / steps, 3) for x in ks["phase_wait_us"]]
        print(json.dumps(out), flush=True)

    try:
        runtime.begin_document()  # warm-up: the kernels' first launches
        runtime.advance_frozen_batch([(b, None) for b in text[:200]])
        if frozen:
            runtime.begin_document()
            timed("frozen", lambda: runtime.advance_frozen_batch([(b, None) for b in text[:frozen]]), frozen)
        if supervised:
            runtime.begin_document()
            steps = [(text[i], text[i + 1]) for i in range(supervised)]
            timed("supervised", lambda: runtime.training_step_batch(steps, native.TRAINING), supervised)
    finally:
        runtime.close()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", default="D")
    ap.add_argument("--no-replay", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain device copy of known size (PMC counter calibration)")
    ap.add_argument("--canonical-steps", nargs=2, type=int, metavar=("FROZEN", "SUPERVISED"),
                    help="time FROZEN prefix steps and SUPERVISED replay-target steps of the canonical runtime "
                         "(kernel time per step) instead of the training benchmark")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration()
    if args.canonical_steps:
        return canonical_steps(args.workload, *args.canonical_steps)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box in this setup has one MI355X, so --gpus {args.gpus} "
              "is not run (stories would be sharded over devices by lane ranges, with the batch-end mean "
              "chained over xGMI; that exchange is not built)", file=sys.stderr)
        return 2

    from leo_amd import native
    from leo_amd.runtime import HipRuntime
    from leo_amd.workload import WORKLOADS, synthetic_stories, workload_model

    w = WORKLOADS[args.workload]
    replay = not args.no_replay
    lanes = w.lanes
    model = workload_model(w)
    total_batches = args.warmup + args.steps
    data, offsets = synthetic_stories(w, total_batches * lanes)
    runtime = HipRuntime(model, device=0, max_lanes=lanes)
    batches = []
    for b in range(total_batches):
        lo, hi = b * lanes, (b + 1) * lanes
        d = data[int(offsets[lo]):int(offsets[hi])].copy()
        o = (offsets[lo:hi + 1] - offsets[lo]).astype("uint64")
        batches.append((d, o))
    for b in range(args.warmup):
        runtime.train_batch_packed(*batches[b], native.TRAINING, replay=replay)
    _device_sync()
    runtime.kernel_stats(reset=True)
    trained = 0
    replay_steps = prefix_steps = 0
    wall = {"story": 0.0, "merge": 0.0, "replay": 0.0}  # host wall clock of each part, summed over the batches
    t0 = time.perf_counter()
    for b in range(args.warmup, total_batches):
        rep = runtime.train_batch_packed(*batches[b], native.TRAINING, replay=replay)
        trained += int(batches[b][1][-1])
        replay_steps += rep.replay_steps
        prefix_steps += rep.replay_prefix_steps
        for k in wall:
            wall[k] += getattr(rep, k + "_seconds")
    _device_sync()
    elapsed = time.perf_counter() - t0
    ks = runtime.kernel_stats()
    bpb = runtime.model().bits_per_byte()
    runtime.close()

    kernel_s = ks["kernel_ms"] / 1e3
    achieved = ks["algorithmic_bytes"] / kernel_s / 1e9 if kernel_s > 0 else 0.0

    def section(name, launches, ms, nbytes, steps):
        gbs = nbytes / (ms / 1e3) / 1e9 if ms > 0 else 0.0
        return {"kernel": name, "launches": launches, "kernel_ms": ms, "algorithmic_bytes": nbytes,
                "lane_steps": steps, "achieved": gbs, "frac": gbs / HBM_PEAK_GBS}

    sections = {
        "story": section("leo_lane_steps (story lanes)", ks["section_launches"][0], ks["section_kernel_ms"][0],
                         ks["section_bytes"][0], ks["section_lane_steps"][0]),
        "replay": section("leo_lane_steps + leo_lane_steps_frozen (canonical runtime)", ks["section_launches"][1],
                          ks["section_kernel_ms"][1], ks["section_bytes"][1], ks["section_lane_steps"][1]),
        "merge": section("leo_merge_candidates + leo_merge_fixed", ks["merge_launches"], ks["merge_ms"], ks["merge_bytes"], 0),
    }
    line = {
        "metric": "trained bytes/sec (FP32, 1 MI355X)",
        "value": trained / elapsed,
        "unit": "bytes/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": elapsed / args.steps * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded Zipf-ASCII stories, seeded synthetic model)",
        "config": {
            "workload": f"{w.name}: {w.neurons} units, fan-in {w.synapses} CSR, 256x{w.fanout} input projection, "
                        f"{lanes} story lanes, replay {'0.30' if replay else 'off'}",
            "stories_per_step": lanes,
            "trained_bytes": trained,
            "replay_steps": replay_steps,
            "replay_prefix_steps": prefix_steps,
            "wall_ms_per_step": {k: v * 1e3 / args.steps for k, v in wall.items()},
            "bits_per_byte": bpb,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(w.name),
            "kernel": "leo_lane_steps + leo_lane_steps_frozen",
            "launches": ks["launches"],
            "kernel_ms_total": ks["kernel_ms"],
            "avg_launch_us": ks["kernel_ms"] * 1e3 / max(ks["launches"], 1),
            "algorithmic_bytes": ks["algorithmic_bytes"],
            "lane_steps": ks["lane_steps"],
            "merge_ms": ks["merge_ms"],
            "sections": sections,
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        d, o = batches[args.warmup]
        line["cpu_baseline"] = cpu_baseline(w, model, d, o, replay)
        line["config"]["cpu_baseline_sample"] = line["cpu_baseline"]["sample"]
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    status = main()
    if status:
        sys.exit(status)
