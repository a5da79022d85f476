#!/usr/bin/env python3
"""Benchmark of the MI355X backend on its headline workload.

Default: the YOLOv8n-shaped graph, u8-quantized (QDQ-folded QLinearConv,
fp16 stem and head 1x1s), batch 32, 640x640, on one GPU through
HipGraphRuntime (its launch list replayed on the backend's streams; --capture
replays one HIP graph instead, which measures slower here: hipGraphLaunch
costs more host and device time than the ~70 launches it replaces).  A step
is one run of the graph over one batch already resident in HBM; `value` is
images/s over exactly --steps steps after --warmup untimed steps, bracketed
by stream synchronisation.

Also prints, on the same JSON line:
  roofline     — the dominant kernel family (most GPU time in one run; the
                 implicit-GEMM launches of all tile shapes are one family):
                 its algorithmic work per launch divided by its mean launch
                 time, measured with HIP events on the backend stream (each
                 launch repeated back to back between one event pair, so the
                 time includes the gap between dispatches), against the
                 MI355X dense peak of its bound;
  cpu_baseline — the oracle (dragonwing-cpu restated in C++) on a bounded
                 sample of the same workload, timed on this host's cores.

Other workloads (--workload): qlinearconv, dwconv, conv_f32, yolov8n_f16.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "images/sec YOLOv8n-shape INT8 640² b32 on 1 MI355X; conv % MFMA/HBM peak"
PEAKS = {  # MI355X dense peaks
    "int8": ("mfma", 5000.0, "TOP/s"),
    "f16": ("mfma", 2500.0, "TFLOP/s"),
    "f32": ("mfma", 157.3, "TFLOP/s"),
    "hbm": ("hbm", 8000.0, "GB/s"),
}


def kernel_bound(kernel: str):
    """The roofline a kernel family is reported against."""
    if kernel.startswith("igemm_i8"):
        return PEAKS["int8"]
    if kernel.startswith("igemm_f16"):
        return PEAKS["f16"]
    if kernel.startswith("direct_conv") or kernel.startswith("stem_pad"):
        return PEAKS["f32"]
    return PEAKS["hbm"]  # the u8 -> f16 1x1 convs (conv1x1_u8_f16) are HBM-bound


def arith_peak(kernel: str):
    """Dense peak (TFLOP/s or TOP/s) of a conv kernel's arithmetic."""
    if kernel.startswith("igemm_i8"):
        return PEAKS["int8"][1]
    if kernel.startswith("igemm_f16") or kernel.startswith("conv1x1"):
        return PEAKS["f16"][1]
    return PEAKS["f32"][1]


def conv_rooflines(launches, ms):
    """Each conv launch against its roofline: the larger of its algorithmic
    work at the dense peak of its arithmetic and its algorithmic bytes at
    8 TB/s is the floor; the fraction is floor / measured time.  Returns the
    per-launch rows and a summary (median, and floor sum / time sum)."""
    rows = []
    for L, t in zip(launches, ms):
        k = L["kernel"]
        if not (k.startswith("igemm") or k.startswith("direct_conv") or k.startswith("stem_pad") or
                k.startswith("dwconv") or k.startswith("conv1x1")):
            continue
        t_mfma = L["work"] / (arith_peak(k) * 1e12) if not k.startswith("dwconv") else 0.0
        t_hbm = L["bytes"] / (PEAKS["hbm"][1] * 1e9)
        floor = max(t_mfma, t_hbm)
        secs = float(t) * 1e-3
        rows.append({"op": L["ops"].split("+")[0], "kernel": k, "us": round(secs * 1e6, 2),
                     "floor_us": round(floor * 1e6, 2), "bound": "mfma" if t_mfma >= t_hbm else "hbm",
                     "frac": round(floor / secs, 4) if secs > 0 else None})
    if not rows:
        return rows, None
    fr = sorted(r["frac"] for r in rows)
    summary = {"launches": len(rows), "median_frac": fr[len(fr) // 2],
               "floor_over_time": round(sum(r["floor_us"] for r in rows) / sum(r["us"] for r in rows), 4),
               "note": "per conv launch: max(work at the dense peak of its arithmetic, bytes at 8 TB/s) / time"}
    return rows, summary


def cpu_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def family(kernel: str) -> str:
    """Kernel family of a launch name: the implicit-GEMM launches of one
    element type are one kernel template whatever their tile shape
    (igemm_i8_c64_p128 -> igemm_i8)."""
    if kernel.startswith("igemm_"):
        return "_".join(kernel.split("_")[:2])
    return kernel


def profile(rts, launches, iters: int, repeat: int):
    """Per-launch milliseconds on the backend stream (each launch enqueued
    `repeat` times back to back between one HIP event pair, averaged over
    `iters` passes: kernel duration plus the dispatch-to-dispatch gap; with
    several runtimes the repeats cycle through their buffer sets), and per
    kernel family: launches, total ms, algorithmic work and bytes."""
    from dragonwing_edge_rs_amd.graph import time_launches_rotated

    acc = None
    for i in range(iters):
        if len(rts) > 1:
            ms = time_launches_rotated(rts, repeat).astype(np.float64)
        else:
            ms = rts[0].time_launches(repeat).astype(np.float64)
        acc = ms if acc is None else acc + ms
    ms = acc / iters
    fam = {}
    for L, t in zip(launches, ms):
        k = family(L["kernel"])
        f = fam.setdefault(k, {"kernel": k, "launches": 0, "ms": 0.0, "work": 0.0, "bytes": 0.0})
        f["launches"] += 1
        f["ms"] += float(t)
        f["work"] += L["work"]
        f["bytes"] += L["bytes"]
    return ms, sorted(fam.values(), key=lambda f: -f["ms"])


def roofline_of(fam):
    bound, peak, unit = kernel_bound(fam["kernel"])
    secs = fam["ms"] * 1e-3
    if bound == "hbm":
        achieved = fam["bytes"] / secs / 1e9
    else:
        achieved = fam["work"] / secs / 1e12
    return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": None, "kernel": fam["kernel"],
            "launches_per_step": fam["launches"], "mean_launch_us": round(fam["ms"] * 1e3 / fam["launches"], 2),
            "work_per_launch": fam["work"] / fam["launches"], "bytes_per_launch": fam["bytes"] / fam["launches"]}


# ---------------------------------------------------------------------------
# CPU baselines (oracle, bounded samples)
# ---------------------------------------------------------------------------
def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline_yolo_int8(info, x_f16, seconds: float):
    from oracle.cpu_graph import CpuGraph
    from dragonwing_edge_rs_amd import yolo

    threads = cpu_threads()
    g1, info1 = yolo.int8_graph_from_ranges(info["ranges"], batch=1, size=info["size"])
    desc = g1.to_dict()

    def sample(int8_threads, secs, most):
        done, t0 = 0, time.perf_counter()
        while True:
            cg = CpuGraph(desc, g1.initializer, threads=threads, int8_threads=int8_threads)
            cg.set_input(info1["input"], x_f16[done % x_f16.shape[0]][None])
            cg.run()
            done += 1
            el = time.perf_counter() - t0
            if el >= secs or done >= most:
                return done, el

    done, el = sample(threads, seconds, 4 * x_f16.shape[0])
    # the reference's own form: conv2d_i8_nhwc has no _mt variant
    # (ops.rs:3086-3142), so its int8 convs run on one thread
    d1, e1 = sample(1, min(seconds, 10.0), x_f16.shape[0])
    return {"value": round(done / el, 3), "unit": "images/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{done} images (cycling through the batch's 32, 640x640) through the oracle's CpuGraph "
                      f"on the same u8 graph "
                      f"at batch 1; int8 convs row-parallel on {threads} threads (bit-identical to the "
                      f"single-threaded conv2d_i8_nhwc form); {el:.1f} s",
            "int8_convs_one_thread": {"value": round(d1 / e1, 3), "unit": "images/s",
                                      "sample": f"{d1} images with the int8 convs on one thread as the "
                                                f"reference runs them (other ops on {threads}); {e1:.1f} s"}}


def cpu_baseline_yolo_f16(info, x_f16, seconds: float):
    from oracle.cpu_graph import CpuGraph
    from dragonwing_edge_rs_amd import yolo

    threads = cpu_threads()
    g1, info1 = yolo.f16_graph(batch=1, size=info["size"])
    desc = g1.to_dict()
    done, t0 = 0, time.perf_counter()
    while True:
        cg = CpuGraph(desc, g1.initializer, threads=threads)
        cg.set_input(info1["input"], x_f16[done % x_f16.shape[0]][None])
        cg.run()
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds or done >= x_f16.shape[0]:
            break
    return {"value": round(done / el, 3), "unit": "images/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{done} of the 32 images through the oracle's CpuGraph (conv2d_fp16_nhwc_mt on "
                      f"{threads} threads); {el:.1f} s"}


def cpu_baseline_qconv(case, seconds: float):
    import oracle

    threads = cpu_threads()
    done, t0 = 0, time.perf_counter()
    while True:
        sl = slice(done % 32, done % 32 + 1)
        oracle.qlinearconv_u8s8(case["x"][sl], case["w"], case["bias"], (2, 2), (1, 1), case["x_scale"],
                                case["x_zp"], case["w_scales"], case["y_scale"], case["y_zp"], threads)
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds or done >= 32:
            break
    return {"value": round(done / el, 3), "unit": "images/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{done} of the 32 images (80x80x128 -> 40x40x256) through the oracle QLinearConv on "
                      f"{threads} threads; {el:.1f} s"}


def cpu_baseline_dwconv(xwb, seconds: float):
    import oracle

    x, w, b = xwb
    threads = cpu_threads()
    done, t0 = 0, time.perf_counter()
    while True:
        sl = slice(done % 32, done % 32 + 1)
        y = oracle.depthwise_fp16(x[sl], w, (1, 1), (1, 1), threads)
        oracle.silu_fp16(oracle.bias_add_f16(y, b))
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds or done >= 32:
            break
    return {"value": round(done / el, 3), "unit": "images/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{done} of the 32 images through depthwise_conv2d_fp16_nhwc_mt + bias + sigmoid/mul "
                      f"on {threads} threads; {el:.1f} s"}


def cpu_baseline_conv_f32(xwb, seconds: float):
    import oracle

    x, w, b = xwb
    threads = cpu_threads()
    done, t0 = 0, time.perf_counter()
    while True:
        oracle.relu_f32(oracle.bias_add_f32(oracle.conv2d_f32_nhwc(x, w, (1, 1), (1, 1), threads), b))
        done += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    return {"value": round(done / el, 3), "unit": "images/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{done} runs of conv2d_f32_nhwc_mt + bias + relu on {threads} threads; {el:.1f} s"}


# ---------------------------------------------------------------------------
# HBM traffic from rocprofv3 counters
# ---------------------------------------------------------------------------
PROBE_BYTES = 256 << 20


def copy_probe(be):
    """One plain copy kernel of PROBE_BYTES read + PROBE_BYTES written: the
    known-size reference for scaling FETCH_SIZE / WRITE_SIZE readings."""
    from dragonwing_edge_rs_amd import ops

    src, dst = be.alloc(PROBE_BYTES), be.alloc(PROBE_BYTES)
    ops.concat_channels_nhwc(be, ops.DTYPE_U8, [src], [PROBE_BYTES >> 10], dst, 1 << 10)
    be.synchronize()
    src.free()
    dst.free()


def read_counter_csv(d: Path):
    import csv

    files = sorted(d.rglob("*counter_collection.csv"))
    if not files:
        raise RuntimeError(f"no counter_collection.csv under {d}")
    rows = {}
    with open(files[0]) as f:
        for r in csv.DictReader(f):
            k = int(r["Dispatch_Id"])
            name, v = r["Kernel_Name"], float(r["Counter_Value"])
            rows[k] = (name, rows[k][1] + v if k in rows else v)
    return [rows[k] for k in sorted(rows)]


def plan_env(launches):
    """The timed plan choices of a runtime (which fused C2f blocks, chained
    pairs, fused head 1x1s, folded upsamples and sibling GEMMs it kept), as the
    environment that makes another process build the same launch list."""
    first = lambda L: L["ops"].split("+")[0]
    return {"DW_PAIR_KEEP": ",".join(first(L) for L in launches if L["kernel"].startswith("igemm_i8_pair")),
            "DW_HEAD_KEEP": ",".join(first(L) for L in launches if L["kernel"].endswith("_head")),
            "DW_C2F_KEEP": ",".join(first(L) for L in launches if L["kernel"].startswith("igemm_i8_c2f")),
            "DW_RESIZE_KEEP": ",".join(L["ops"].split("+")[-1] for L in launches if L["kernel"].endswith("_up")),
            "DW_SIB_KEEP": ",".join(first(L) for L in launches if L["kernel"].endswith("_sib"))}


def measure_traffic(workload: str, launches, timeout: float = 240.0):
    """Per-launch HBM bytes: two rocprofv3 counter passes (FETCH_SIZE, then
    WRITE_SIZE) over a child run of this workload that brackets one graph
    run between two copy probes; each counter is scaled by what it reads for
    the second probe.  The child builds this run's plan (plan_env).  Returns
    (fetch_bytes[], write_bytes[], scales) in launch order, or raises."""
    import shutil
    import signal
    import subprocess
    import tempfile

    exe = shutil.which("rocprofv3")
    if not exe:
        raise RuntimeError("rocprofv3 not found")
    base = Path(tempfile.mkdtemp(prefix="dw_traffic_", dir="/tmp"))
    per, scales = {}, {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        d = base / counter
        cmd = [exe, "--pmc", counter, "--output-format", "csv", "-d", str(d), "-o", "run", "--",
               sys.executable, str(ROOT / "bench.py"), "--workload", workload, "--traffic-child"]
        p = subprocess.Popen(cmd, cwd="/tmp", env=dict(os.environ, TMPDIR="/tmp", **plan_env(launches)),
                             stdout=subprocess.DEVNULL,
                             stderr=subprocess.DEVNULL, start_new_session=True)
        try:
            p.wait(timeout=timeout)
        except subprocess.TimeoutExpired:
            os.killpg(p.pid, signal.SIGKILL)
            p.wait()
            raise RuntimeError(f"{counter} pass timed out")
        rows = read_counter_csv(d)
        copies = [i for i, (n, _) in enumerate(rows) if "copy_channels" in n]
        if len(copies) < 2:
            raise RuntimeError(f"{counter}: copy probes not found")
        b = copies[-1]
        a = b - len(launches) - 1
        if a < 0 or "copy_channels" not in rows[a][0]:
            raise RuntimeError(f"{counter}: {b - copies[-2] - 1} dispatches between the probes, "
                               f"{len(launches)} launches expected")
        scale = (PROBE_BYTES / 1024.0) / rows[b][1]
        per[counter] = [rows[i][1] * scale * 1024.0 for i in range(a + 1, b)]
        scales[counter] = round(scale, 4)
    shutil.rmtree(base, ignore_errors=True)
    return per["FETCH_SIZE"], per["WRITE_SIZE"], scales


# ---------------------------------------------------------------------------
def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=0,
                    help="timed steps (default: 3000 for the graphs, 10000 for the single-op workloads: a "
                         "few seconds of GPU work, long enough for an outside utilisation sampler to see it)")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="yolov8n_int8",
                    choices=["yolov8n_int8", "yolov8n_f16", "qlinearconv", "dwconv", "conv_f32"])
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--profile-iters", type=int, default=3)
    ap.add_argument("--profile-repeat", type=int, default=10,
                    help="back-to-back repeats of each launch per timing pass")
    ap.add_argument("--capture", action="store_true", help="replay one captured HIP graph per step")
    ap.add_argument("--dump-launches", default="", help="write per-launch timings (JSON lines) to this file")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 counter passes that measure roofline.traffic")
    ap.add_argument("--traffic-child", action="store_true", help=argparse.SUPPRESS)
    ap.add_argument("--traffic-probe", action="store_true",
                    help="end with one plain 256 MiB device copy (copy_channels kernel), the known-size "
                         "reference for scaling FETCH_SIZE / WRITE_SIZE counters of the same run")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this backend runs on one GPU; --gpus {args.gpus} is not supported "
              f"(the batch would shard data-parallel across GPUs with no exchange).", file=sys.stderr)
        sys.exit(2)

    if args.steps <= 0:
        args.steps = 3000 if args.workload.startswith("yolov8n") else 10000
    import __graft_entry__

    dw = __graft_entry__.import_pkg()
    from dragonwing_edge_rs_amd import workloads
    from dragonwing_edge_rs_amd.graph import HipGraphRuntime

    be = dw.Backend(0)
    wl = args.workload
    rotate = 1
    t_setup = time.perf_counter()
    if wl == "yolov8n_int8":
        g, inputs, outs, work, extra = workloads.yolov8n_int8(be)
        config = {"workload": "YOLOv8n-shaped graph, u8 QDQ (QLinearConv, fp16 stem + head 1x1s), "
                              "batch 32, 640x640, calibrated on 16 uniform images",
                  "batch": 32, "size": 640, "convs": extra["convs"], "params": extra["params"]}
        dtype = "int8"
    elif wl == "yolov8n_f16":
        g, inputs, outs, work, extra = workloads.yolov8n_f16()
        config = {"workload": "YOLOv8n-shaped graph, fp16, batch 32, 640x640", "batch": 32, "size": 640,
                  "convs": extra["convs"], "params": extra["params"]}
        dtype = "f16"
    elif wl == "qlinearconv":
        g, inputs, outs, work, extra = workloads.qlinearconv()
        config = {"workload": "QLinearConv u8xs8->u8, N=32, 80x80x128 -> 40x40x256, 3x3 s2 p1", "batch": 32}
        dtype = "int8"
        rotate = 8  # 8 x 39.6 MB > 256 MB Infinity Cache
    elif wl == "dwconv":
        g, inputs, outs, work, extra = workloads.dwconv()
        config = {"workload": "depthwise 3x3 fp16 + bias + SiLU, N=32, C=384, 40x40", "batch": 32}
        dtype = "f16"
        rotate = 4  # 4 x 78.7 MB > 256 MB Infinity Cache
    else:
        g, inputs, outs, work, extra = workloads.conv_f32()
        config = {"workload": "Conv2d fp32 + bias + ReLU, N=1, 64->64, 56x56, 3x3 s1 p1", "batch": 1}
        dtype = "f32"
    rts = [HipGraphRuntime(g, be) for _ in range(rotate)]
    for rt in rts:
        for k, v in inputs.items():
            rt.set_input_bytes(k, v)
        if args.capture:
            rt.enable_capture(True)
    t_setup = time.perf_counter() - t_setup
    images = work["images"]
    if args.traffic_child:
        # counted run: probe, one graph run, probe (nothing else on the GPU)
        rts[0].run()
        be.synchronize()
        copy_probe(be)
        rts[0].run()
        be.synchronize()
        copy_probe(be)
        return

    for i in range(args.warmup):
        rts[i % rotate].run()
    be.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        rts[i % rotate].run()
    be.synchronize()
    el = time.perf_counter() - t0
    ms_per_step = el * 1e3 / args.steps
    value = images * args.steps / el

    launches = rts[0].launches()
    ms, fams = profile(rts, launches, args.profile_iters, args.profile_repeat)
    if args.dump_launches:
        with open(args.dump_launches, "w") as f:
            for L, t in zip(launches, ms):
                f.write(json.dumps(dict(L, ms=round(float(t), 5))) + "\n")
    dom = fams[0]
    roof = roofline_of(dom)
    roof["timing"] = ("each launch repeated back to back between HIP events" +
                      (", cycling through %d buffer sets (more than the Infinity Cache holds)" % rotate
                       if rotate > 1 else ""))
    kernels = []
    for f in fams[:8]:
        r = roofline_of(f)
        kernels.append({"kernel": f["kernel"], "launches": f["launches"], "ms": round(f["ms"], 4),
                        "achieved": r["achieved"], "unit": r["unit"], "frac": r["frac"]})

    cpu = None
    if not args.no_cpu_baseline:
        if wl == "yolov8n_int8":
            cpu = cpu_baseline_yolo_int8(extra, inputs[extra["input"]], args.cpu_seconds)
        elif wl == "yolov8n_f16":
            cpu = cpu_baseline_yolo_f16(extra, inputs[extra["input"]], args.cpu_seconds)
        elif wl == "qlinearconv":
            cpu = cpu_baseline_qconv(extra, args.cpu_seconds)
        elif wl == "dwconv":
            cpu = cpu_baseline_dwconv(extra, args.cpu_seconds)
        else:
            cpu = cpu_baseline_conv_f32(extra, args.cpu_seconds)

    line = {
        "metric": METRIC if wl == "yolov8n_int8" else f"images/sec {wl} on 1 MI355X",
        "value": round(value, 2),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": "synthetic (seeded LCG inputs, random-init weights with BN folded)",
        "config": config,
        "roofline": roof,
        "cpu_baseline": cpu,
        "kernels": kernels,
        "gpu_ms_sum_of_launches": round(float(ms.sum()), 4),
        "setup_s": round(t_setup, 1),
    }
    conv_rows, conv_summary = conv_rooflines(launches, ms)
    if conv_summary:
        line["convs"] = conv_summary
    if args.dump_launches:
        with open(args.dump_launches + ".convs.json", "w") as f:
            json.dump(conv_rows, f, indent=0)
    arena, unshared = rts[0].activation_bytes()
    line["activation_bytes"] = {"arena": arena, "without_reuse": unshared}
    if not args.no_traffic:
        try:
            fetch, write, scales = measure_traffic(wl, launches)
            idx = [i for i, L in enumerate(launches) if family(L["kernel"]) == dom["kernel"]]
            fb = sum(fetch[i] for i in idx) / len(idx)
            wb = sum(write[i] for i in idx) / len(idx)
            roof["traffic"] = round(fb + wb)
            roof["traffic_fetch"] = round(fb)
            roof["traffic_write"] = round(wb)
            roof["traffic_over_algorithmic"] = round((fb + wb) / roof["bytes_per_launch"], 3)
            roof["traffic_source"] = ("rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes over one graph run, "
                                      "per-dispatch KiB scaled by the readings of a 256 MiB copy (scales %s)"
                                      % scales)
            # every listed family: measured HBM bytes per launch against its algorithmic bytes
            for k in kernels:
                fi = [i for i, L in enumerate(launches) if family(L["kernel"]) == k["kernel"]]
                alg = sum(launches[i]["bytes"] for i in fi) / len(fi)
                t = sum(fetch[i] + write[i] for i in fi) / len(fi)
                k["traffic_per_launch"] = round(t)
                k["traffic_over_algorithmic"] = round(t / alg, 3) if alg > 0 else None
        except Exception as e:  # the counters are optional: the line stands without them
            roof["traffic_source"] = f"not measured: {e}"
    if args.traffic_probe:
        copy_probe(be)
        line["traffic_probe_bytes"] = {"read": PROBE_BYTES, "write": PROBE_BYTES}
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
