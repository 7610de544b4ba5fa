#!/usr/bin/env python3
"""Throughput benchmark of the MI355X backend.

The LAST stdout line is the headline JSON record (under 8 KB); detail
records (per-configuration kernel tables, pass rates, host pipeline timings,
CPU sample descriptions) come first, one JSON line each, as
``{"detail": name, "data": ...}``.

Workload (the headline configuration that fits one GPU): the PP-OCRv6
medium detector, fp32, batch 8 of 3x416x736 seeded-pixel images with seeded
weights at the reference tensor shapes.  A step is one pass of the detector
over the batch; inputs are resident in HBM before the timed region, which is
``--steps`` back-to-back passes between two stream synchronisations.

Alongside ``value`` the line carries:
* ``roofline``: the dominant kernel (most device time per step), its
  algorithmic FLOPs (2 x MACs) or bytes per step over its HIP-event-timed
  duration (events recorded on the stream the kernels run on), against the
  MI355X peak of the roof it runs under (fp32 matrix 157.3 TFLOP/s, bf16
  matrix 2.5 PFLOP/s, fp32 vector 78.6 TFLOP/s without packed fp32, HBM
  8 TB/s; a compute kernel whose algorithmic FLOPs per byte stay below that
  compute peak's ridge point is measured in bytes against HBM, the roofline
  model's lower roof, see bound_of); ``traffic`` is its measured HBM bytes per launch from the
  committed counter summary, when one covers this kernel and workload;
* (detail line) the same measure for the twelve kernel instances with the
  most device time (the depthwise and elementwise ones against HBM);
* ``pass``: the whole pass's algorithmic FLOPs and bytes per step over the
  step time;
* ``cpu_baseline``: the C++ restatement of the reference CPU path (the
  parity oracle) timed on this host on a bounded sample of the same
  workload, at the reference's default thread count (min(cores, 4),
  src/cpu/model.rs:19-27); ``others`` holds the same at every CPU this
  process may use and for the tiny and medium recognizers;
* ``also``: the other benchmark configurations, measured after the timed
  region: value, step time and the dominant kernel's roofline fraction
  (their full records, with pass rates and kernel tables, are detail lines).
"""

import argparse
import json
import os
import pathlib
import sys
import tempfile
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "ppocr-rs_amd"))

import numpy as np  # noqa: E402

import ppocr_hip  # noqa: E402
import seeded  # noqa: E402

METRIC = "detector images/s @416×736 + rec lines/s @48×320; % HBM/MFMA roofline"
PEAK_F32_TFLOPS = 157.3
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
# fp32 FMAs on the vector ALU without packed-fp32 instructions (the HIP code
# is compiled without them): 256 CUs x 4 SIMDs x 16 lanes x 2 FLOP x 2.4 GHz.
PEAK_VALU_F32_TFLOPS = 78.6
TMP = pathlib.Path(tempfile.gettempdir()) / "ppocr_bench_models"


def weights(kind, size):
    TMP.mkdir(parents=True, exist_ok=True)
    gain, head_gain = seeded.DEFAULT_GAINS[(kind, size)]
    path = TMP / f"{kind}_{size}_g{gain}_{head_gain}.safetensors"
    if not path.exists():
        seeded.write_weights(path, kind, size, seed=1 if kind == "det" else 2)
    return path


def load(gpu, kind, size, shape, precision="f32", greedy=False):
    if kind == "det":
        return ppocr_hip.Detector.load(gpu, weights(kind, size), size, shape, precision=precision)
    return ppocr_hip.Recognizer.load(gpu, weights(kind, size), size, shape, precision=precision, greedy=greedy)


def inputs(kind, shape, seed=7):
    return seeded.seeded_batch(shape[0], shape[2], shape[3], seed, detector=(kind == "det"))


def throughput(model, x, warmup, steps):
    total_ms = model.benchmark_stream(x, warmup, steps)
    return total_ms


def kernel_groups(stats):
    """Per-step device time and algorithmic work of each kernel instance."""
    groups = {}
    for s in stats:
        g = groups.setdefault(s["kernel"], {"ms": 0.0, "flops": 0.0, "bytes": 0.0, "launches": 0, "bound": s["bound"]})
        g["ms"] += s["avg_ms"]
        g["flops"] += s["flops"]
        g["bytes"] += s["bytes"]
        g["launches"] += 1
    return groups


def compute_peak(bound, precision="f32"):
    """Peak TFLOP/s of a compute roof (matrix or vector)."""
    if bound == "mfma":
        return PEAK_BF16_TFLOPS if precision == "bf16" else PEAK_F32_TFLOPS
    return PEAK_VALU_F32_TFLOPS


def bound_of(g, precision="f32"):
    """The roof a kernel group runs under (the roofline model): the compute
    roof its kernel is built for (matrix cores or vector ALUs) when its
    arithmetic intensity, algorithmic FLOPs per algorithmic HBM byte, reaches
    that roof's ridge point (peak FLOP/s over the 8 TB/s of HBM; 19.7 FLOP/B
    for fp32 matrix products, 312.5 for bf16); below the ridge HBM is the
    lower roof, and the group is measured against it (achieved bytes / 8 TB/s
    equals achieved FLOPs over the attainable intensity x bandwidth)."""
    if g["bound"] not in ("mfma", "valu") or g["bytes"] <= 0:
        return g["bound"]
    ridge = compute_peak(g["bound"], precision) * 1e12 / (PEAK_HBM_GBS * 1e9)
    return g["bound"] if g["flops"] / g["bytes"] >= ridge else "hbm"


def rate(g, precision="f32"):
    """(achieved, peak, unit) of a kernel group against its roof (bound_of)."""
    secs = g["ms"] * 1e-3
    bound = bound_of(g, precision)
    if bound in ("mfma", "valu"):
        return g["flops"] / secs / 1e12, compute_peak(bound, precision), "TFLOP/s"
    return g["bytes"] / secs / 1e9, PEAK_HBM_GBS, "GB/s"


def kernel_table(stats, top=12, precision="f32"):
    """The `top` kernel instances by device time, each against its roofline."""
    groups = kernel_groups(stats)
    total_ms = sum(v["ms"] for v in groups.values())
    rows = []
    for name, g in sorted(groups.items(), key=lambda kv: -kv[1]["ms"])[:top]:
        achieved, peak, unit = rate(g, precision)
        rows.append({"kernel": name, "bound": bound_of(g, precision),
                     "launches_per_step": g["launches"], "ms_per_step": round(g["ms"], 4),
                     "share_of_device_time": round(g["ms"] / total_ms, 3) if total_ms else None,
                     "achieved": round(achieved, 2), "unit": unit, "frac": round(achieved / peak, 3)})
    return rows


def roofline(stats, key, precision="f32"):
    """Dominant kernel instance: the one with the most device time per step."""
    groups = kernel_groups(stats)
    name, g = max(groups.items(), key=lambda kv: kv[1]["ms"])
    achieved, peak, unit = rate(g, precision)
    total_ms = sum(v["ms"] for v in groups.values())
    return {
        "bound": bound_of(g, precision),
        "achieved": round(achieved, 3),
        "peak": peak,
        "unit": unit,
        "frac": round(achieved / peak, 4),
        "traffic": traffic_for(key, name),
        "kernel": name,
        "launches_per_step": g["launches"],
        "avg_launch_ms": round(g["ms"] / g["launches"], 5),
        "flops_per_launch": g["flops"] / g["launches"],
        "bytes_per_launch": g["bytes"] / g["launches"],
        "share_of_device_time": round(g["ms"] / total_ms, 3) if total_ms else None,
    }


def traffic_for(key, kernel):
    """HBM bytes per launch of `kernel` in workload `key` from the committed
    counter summary ``profiles/traffic_<key>.txt``.

    A summary is written from two rocprofv3 --pmc runs of this benchmark
    (FETCH_SIZE, WRITE_SIZE, KiB per dispatch), each scaled by the same
    counter's reading for a copy kernel of known size (``--copy-calibration``).
    Returns None when no summary covers this kernel.
    """
    path = ROOT / "profiles" / f"traffic_{key}.txt"
    if not path.exists():
        return None
    fields = {}
    for line in path.read_text().splitlines():
        if ":" in line and not line.startswith("#"):
            k, v = line.split(":", 1)
            fields[k.strip()] = v.strip()
    if fields.get("kernel") != kernel:
        return None
    try:
        return float(fields["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def copy_calibration(mib=256, reps=5):
    """A plain device copy of known size (y = -x over `mib` MiB of fp32),
    run under rocprofv3 --pmc to scale FETCH_SIZE / WRITE_SIZE to bytes."""
    import torch

    n = mib * (1 << 20) // 4
    x = torch.ones(n, device="cuda", dtype=torch.float32)
    y = torch.empty_like(x)
    for _ in range(reps):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration": {"bytes_read": n * 4, "bytes_written": n * 4, "launches": reps}}))


def usable_cpus():
    """CPUs this process may run on (its affinity mask, capped by
    OMP_NUM_THREADS when that is set), and a description of how it was found."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS", "")
    n = min(affinity, int(omp)) if omp.isdigit() and int(omp) > 0 else affinity
    return n, f"os.cpu_count()={os.cpu_count()}, affinity={affinity}, OMP_NUM_THREADS={omp or 'unset'}"


def cpu_time(kind, size, threads, budget_s):
    """Single-item passes of the oracle for `budget_s` seconds (one warm-up)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    oracle.set_threads(threads)
    model = oracle.Model(kind, weights(kind, size), size)
    one = (1, 3, 416, 736) if kind == "det" else (1, 3, 48, 320)
    x = inputs(kind, one)
    model.forward(x)  # warm-up
    runs, t0 = 0, time.perf_counter()
    while True:
        model.forward(x)
        runs += 1
        el = time.perf_counter() - t0
        if el >= budget_s or runs >= 200:
            break
    unit = "images/s" if kind == "det" else "lines/s"
    what = "detector" if kind == "det" else "recognizer"
    return {"value": round(runs / el, 3), "unit": unit, "cores": threads, "kind": "port",
            "sample": f"{runs} single-{'image' if kind == 'det' else 'line'} passes ({el:.1f} s) of the {size} "
                      f"{what} at {one}, C++ restatement of the reference CPU path (fp32, OpenMP, "
                      f"{threads} threads)"}


def cpu_baseline(kind, size):
    """The oracle at the reference's default thread count, min(cores, 4)
    (src/cpu/model.rs:19-27), with the same at every usable CPU and for the
    tiny and medium recognizers under ``others`` (value, unit, threads and
    workload only; the full sample descriptions go to an earlier line)."""
    cpus, how = usable_cpus()
    base = cpu_time(kind, size, min(cpus, 4), 10.0)
    base["cpus"] = how
    others = [("det", size, cpu_time(kind, size, cpus, 8.0)), ("rec", "tiny", cpu_time("rec", "tiny", min(cpus, 4), 3.0)),
              ("rec", "tiny", cpu_time("rec", "tiny", cpus, 3.0)),
              ("rec", "medium", cpu_time("rec", "medium", min(cpus, 4), 4.0))]
    emit("cpu_baseline_samples", [o["sample"] for _, _, o in others])
    base["others"] = [{"workload": f"{sz} {'detector 1x3x416x736' if k == 'det' else 'recognizer 1x3x48x320'}",
                       "value": o["value"], "unit": o["unit"], "cores": o["cores"]} for k, sz, o in others]
    return base


def emit(name, payload):
    """One detail line (JSON) on stdout ahead of the headline line."""
    print(json.dumps({"detail": name, "data": payload}), flush=True)


def config_key(kind, size, shape, precision, greedy=False):
    return f"{size}_{kind}_{shape[0]}x{shape[2]}x{shape[3]}_{precision}" + ("_greedy" if greedy else "")


HEADLINE = ("det", "medium", (8, 3, 416, 736), "f32")
HEADLINE_KEY = config_key(*HEADLINE)


def pass_rates(stats, ms_per_step, precision):
    """Whole-pass algorithmic FLOP and byte rates per step."""
    flops = sum(s["flops"] for s in stats)
    nbytes = sum(s["bytes"] for s in stats)
    secs = ms_per_step * 1e-3
    peak = PEAK_BF16_TFLOPS if precision == "bf16" else PEAK_F32_TFLOPS
    return {"gflop_per_step": round(flops / 1e9, 3), "mb_per_step": round(nbytes / 1e6, 2),
            "tflops": round(flops / secs / 1e12, 3), "frac_of_matrix_peak": round(flops / secs / 1e12 / peak, 4),
            "gbs": round(nbytes / secs / 1e9, 1), "frac_of_hbm": round(nbytes / secs / 1e9 / PEAK_HBM_GBS, 4),
            "kernels_per_step": len(stats)}


def measure(gpu, kind, size, shape, precision, greedy, warmup, steps, top=5):
    """Throughput, dominant-kernel roofline and pass rates of one configuration."""
    key = config_key(kind, size, shape, precision, greedy)
    m = load(gpu, kind, size, shape, precision, greedy)
    try:
        x = inputs(kind, shape)
        ms = throughput(m, x, warmup, steps)
        stats = m.profile(x, runs=3)
    finally:
        m.close()
    unit = "images/s" if kind == "det" else "lines/s"
    return {"value": round(shape[0] * steps / (ms / 1e3), 2), "unit": unit, "ms_per_step": round(ms / steps, 4),
            "roofline": roofline(stats, key, precision), "pass": pass_rates(stats, ms / steps, precision),
            "kernels": kernel_table(stats, top, precision)}


ALSO_CONFIGS = [
    ("det", "tiny", (1, 3, 416, 736), "f32"),
    ("det", "small", (1, 3, 416, 736), "f32"),
    ("det", "small", (8, 3, 416, 736), "f32"),
    ("det", "medium", (1, 3, 416, 736), "f32"),
    ("det", "tiny", (1, 3, 832, 1472), "f32"),
    ("rec", "tiny", (1, 3, 48, 320), "f32"),
    ("rec", "small", (1, 3, 48, 320), "f32"),
    ("rec", "medium", (1, 3, 48, 320), "f32"),
    ("rec", "tiny", (64, 3, 48, 320), "f32"),
    ("rec", "small", (64, 3, 48, 320), "f32"),
    ("rec", "medium", (256, 3, 48, 320), "f32"),
    ("det", "medium", (1, 3, 416, 736), "bf16"),
    ("det", "medium", (8, 3, 416, 736), "bf16"),
    ("rec", "medium", (256, 3, 48, 320), "bf16"),
    # Recognizers with the classifier fused with greedy CTC step decoding
    # (per-step class + probability instead of [N, T, V] probabilities).
    ("rec", "tiny", (64, 3, 48, 320), "f32", "greedy"),
    ("rec", "medium", (256, 3, 48, 320), "f32", "greedy"),
    ("rec", "medium", (256, 3, 48, 320), "bf16", "greedy"),
]


def also(gpu, warmup, steps):
    out = {}
    for kind, size, shape, precision, *mode in ALSO_CONFIGS:
        greedy = mode == ["greedy"]
        key = config_key(kind, size, shape, precision, greedy)
        try:
            out[key] = measure(gpu, kind, size, shape, precision, greedy, warmup, steps)
        except Exception as e:  # report, keep going
            out[key] = {"error": str(e)}
    return out


def only(key, warmup, steps):
    """Runs one configuration's timed loop alone (for rocprofv3 runs)."""
    gpu = ppocr_hip.Gpu(0)
    for kind in ("det", "rec"):
        for size in ("tiny", "small", "medium"):
            for precision in ("f32", "bf16"):
                for greedy in (False, True):
                    for n, h, w in ((1, 416, 736), (8, 416, 736), (1, 832, 1472), (1, 48, 320), (64, 48, 320),
                                    (256, 48, 320)):
                        shape = (n, 3, h, w)
                        if config_key(kind, size, shape, precision, greedy) != key:
                            continue
                        m = load(gpu, kind, size, shape, precision, greedy)
                        ms = throughput(m, inputs(kind, shape), warmup, steps)
                        m.close()
                        gpu.close()
                        print(json.dumps({"config": key, "ms_per_step": round(ms / steps, 4)}), flush=True)
                        return
    gpu.close()
    raise SystemExit(f"unknown configuration {key}")


def pipeline(gpu, reps=20):
    """End-to-end calls with host buffers (wall clock, PCIe included): the
    detector with the device DB postprocess against the detector returning its
    probability map, and the OCR engine on a 960x540 synthetic page."""
    out = {}
    shape = (1, 3, 416, 736)
    det = load(gpu, "det", "tiny", shape)
    x = inputs("det", shape)
    transforms = [(736, 416, 736, 416)]
    det.forward(x)
    det.detect(x, transforms, binary_threshold=0.62, box_threshold=0.0)
    t0 = time.perf_counter()
    for _ in range(reps):
        det.forward(x)
    t1 = time.perf_counter()
    for _ in range(reps):
        n = len(det.detect(x, transforms, binary_threshold=0.62, box_threshold=0.0)[0])
    t2 = time.perf_counter()
    det.close()
    out["tiny_det_1x416x736_forward_map_to_host_ms"] = round((t1 - t0) / reps * 1e3, 3)
    out["tiny_det_1x416x736_detect_on_device_ms"] = round((t2 - t1) / reps * 1e3, 3)
    out["tiny_det_1x416x736_detections"] = n
    dictionary = [f"<{i}>" for i in range(1, 6906)]
    img = seeded.seeded_rgb(540, 960, 23, pattern="blocks")
    for label, opts in [("default", {}), ("thr0.62", dict(binary_threshold=0.62, box_threshold=0.0))]:
        engine = ppocr_hip.OcrEngine.load(gpu, weights("det", "tiny"), weights("rec", "tiny"), dictionary, **opts)
        r = engine.recognize(img)  # warm: loads and captures every plan
        t0 = time.perf_counter()
        for _ in range(5):
            r = engine.recognize(img)
        el = (time.perf_counter() - t0) / 5
        engine.close()
        out[f"engine_tiny_960x540_{label}"] = {"ms_per_image": round(el * 1e3, 3), "lines": len(r.lines)}
    return out


def compact_also(extra):
    """Per configuration only value, step time and the dominant kernel's
    roofline fraction: the full records go to earlier detail lines."""
    out = {}
    for key, r in extra.items():
        if "error" in r:
            out[key] = {"error": r["error"][:120]}
            continue
        out[key] = {"value": r["value"], "unit": r["unit"], "ms_per_step": r["ms_per_step"],
                    "frac": r["roofline"]["frac"]}
    return out


def headline(value, steps, warmup, ms_per_step, shape, roof, pass_, cpu=None, extra=None):
    """The last stdout line: the metric, its roofline and CPU baseline, and a
    compact summary of the other configurations (kept well under 8 KB so a
    tail of the output always holds it whole)."""
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded uniform RGB8 pixels (BGR-normalised as the reference preprocess), "
                "seeded weights at the reference tensor names/shapes",
        "config": {"workload": "PP-OCRv6 medium detector, fp32, batch 8, input 8x3x416x736",
                   "model_size": "medium", "batch": shape[0], "height": shape[2], "width": shape[3]},
        "roofline": roof,
        "pass": pass_,
    }
    if cpu is not None:
        line["cpu_baseline"] = cpu
    if extra is not None:
        line["also"] = compact_also(extra)
    return json.dumps(line, separators=(",", ":"))


def db_profile(reps=10):
    """The tiny detector's forward + device DB postprocess at 416x736 with the
    postprocess's per-step breakdown (PPOCR_HIP_DB_PROFILE: host steps by
    wall clock, kernels by HIP events; the library prints one JSON line per
    call on stderr) for a page of ~9000 components cut to 1000 detections and
    for the default thresholds, next to the forward with the map read back."""
    os.environ["PPOCR_HIP_DB_PROFILE"] = "1"
    gpu = ppocr_hip.Gpu(0)
    shape = (1, 3, 416, 736)
    det = load(gpu, "det", "tiny", shape)
    x = inputs("det", shape)
    tr = [(736, 416, 736, 416)]
    for thr, box in ((0.5, 0.6), (0.2, 0.4)):
        for _ in range(3):
            d = det.detect(x, tr, binary_threshold=thr, box_threshold=box)
        t0 = time.perf_counter()
        for _ in range(reps):
            d = det.detect(x, tr, binary_threshold=thr, box_threshold=box)
        t1 = time.perf_counter()
        for _ in range(reps):
            det.forward(x)
        t2 = time.perf_counter()
        print(json.dumps({"binary_threshold": thr, "box_threshold": box, "detections": len(d[0]),
                          "detect_ms": round((t1 - t0) / reps * 1e3, 3),
                          "forward_map_to_host_ms": round((t2 - t1) / reps * 1e3, 3)}), flush=True)
    det.close()
    gpu.close()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-extra", action="store_true", help="skip the other configurations")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a known-size copy kernel (for rocprofv3 counter scaling)")
    ap.add_argument("--only", metavar="KEY", help="run only this configuration's timed loop (rocprofv3 runs)")
    ap.add_argument("--db-profile", action="store_true",
                    help="only the device DB postprocess breakdown (JSON lines on stdout and stderr)")
    args = ap.parse_args()
    if args.db_profile:
        db_profile()
        return
    if args.copy_calibration:
        copy_calibration()
        return
    if args.only:
        only(args.only, args.warmup, args.steps)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: the detector/recognizer path has no multi-GPU form in this library "
              "(independent images shard across GPUs without communication); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    kind, size, shape, precision = HEADLINE
    gpu = ppocr_hip.Gpu(0)
    model = load(gpu, kind, size, shape)
    x = inputs(kind, shape)
    total_ms = throughput(model, x, args.warmup, args.steps)
    ms_per_step = total_ms / args.steps
    value = shape[0] * args.steps / (total_ms / 1e3)
    stats = model.profile(x, runs=max(3, min(args.steps, 10)))
    roof = roofline(stats, HEADLINE_KEY, precision)
    model.close()
    emit(HEADLINE_KEY + "_kernels", kernel_table(stats))

    cpu = None if args.no_cpu else cpu_baseline(kind, size)
    extra = None
    if not args.no_extra:
        extra = also(gpu, args.warmup, max(5, args.steps // 2))
        for key, r in extra.items():
            emit(key, r)
        emit("pipeline", pipeline(gpu))
    gpu.close()
    print(headline(value, args.steps, args.warmup, ms_per_step, shape, roof,
                   pass_rates(stats, ms_per_step, precision), cpu, extra), flush=True)


if __name__ == "__main__":
    main()
