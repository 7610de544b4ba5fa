#!/usr/bin/env python3
"""Throughput benchmark of the MI355X backend (one JSON line on stdout).

Workload (the headline configuration that fits one GPU): the PP-OCRv6
medium detector, fp32, batch 8 of 3x416x736 seeded-pixel images with seeded
weights at the reference tensor shapes.  A step is one pass of the detector
over the batch; inputs are resident in HBM before the timed region, which is
``--steps`` back-to-back passes between two stream synchronisations.

Alongside ``value`` the line carries:
* ``roofline``: the dominant kernel (most device time per step), its
  algorithmic FLOPs (2 x MACs) or bytes per step over its HIP-event-timed
  duration (events recorded on the stream the kernels run on), against the
  MI355X peak (fp32 matrix 157.3 TFLOP/s, HBM 8 TB/s);
* ``kernels``: the same measure for the twelve kernel instances with the
  most device time (the depthwise and elementwise ones against HBM);
* ``cpu_baseline``: the C++ restatement of the reference CPU path (the
  parity oracle) timed on this host on a bounded sample of the same workload;
* ``also``: the other benchmark configurations, measured after the timed
  region.
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
PEAK_HBM_GBS = 8000.0
# fp32 FMAs on the vector ALU without packed-fp32 instructions (this build
# disables them): 256 CUs x 4 SIMDs x 16 lanes x 2 FLOP x 2.4 GHz.
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


def rate(g):
    """(achieved, peak, unit) of a kernel group against its bound's peak."""
    secs = g["ms"] * 1e-3
    if g["bound"] == "mfma":
        return g["flops"] / secs / 1e12, PEAK_F32_TFLOPS, "TFLOP/s"
    if g["bound"] == "valu":
        return g["flops"] / secs / 1e12, PEAK_VALU_F32_TFLOPS, "TFLOP/s"
    return g["bytes"] / secs / 1e9, PEAK_HBM_GBS, "GB/s"


def kernel_table(stats, top=12):
    """The `top` kernel instances by device time, each against its roofline."""
    groups = kernel_groups(stats)
    total_ms = sum(v["ms"] for v in groups.values())
    rows = []
    for name, g in sorted(groups.items(), key=lambda kv: -kv[1]["ms"])[:top]:
        achieved, peak, unit = rate(g)
        rows.append({"kernel": name, "bound": g["bound"],
                     "launches_per_step": g["launches"], "ms_per_step": round(g["ms"], 4),
                     "share_of_device_time": round(g["ms"] / total_ms, 3) if total_ms else None,
                     "achieved": round(achieved, 2), "unit": unit, "frac": round(achieved / peak, 3)})
    return rows


def roofline(stats):
    """Dominant kernel instance: the one with the most device time per step."""
    groups = kernel_groups(stats)
    name, g = max(groups.items(), key=lambda kv: kv[1]["ms"])
    achieved, peak, unit = rate(g)
    total_ms = sum(v["ms"] for v in groups.values())
    return {
        "bound": g["bound"],
        "achieved": round(achieved, 3),
        "peak": peak,
        "unit": unit,
        "frac": round(achieved / peak, 4),
        "traffic": traffic_for(name),
        "kernel": name,
        "launches_per_step": g["launches"],
        "avg_launch_ms": round(g["ms"] / g["launches"], 5),
        "flops_per_launch": g["flops"] / g["launches"],
        "bytes_per_launch": g["bytes"] / g["launches"],
        "share_of_device_time": round(g["ms"] / total_ms, 3) if total_ms else None,
    }


TRAFFIC_FILE = ROOT / "profiles" / "dominant_kernel_traffic.txt"


def traffic_for(kernel):
    """HBM bytes per launch of `kernel` from the committed counter summary.

    The summary is written from two rocprofv3 --pmc runs of this benchmark
    (FETCH_SIZE, WRITE_SIZE, KiB per dispatch), each scaled by the same
    counter's reading for a copy kernel of known size (``--copy-calibration``).
    Returns None when the summary covers a different kernel.
    """
    if not TRAFFIC_FILE.exists():
        return None
    fields = {}
    for line in TRAFFIC_FILE.read_text().splitlines():
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


def cpu_baseline(kind, size, shape, budget_s=12.0):
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    threads = min(os.cpu_count() or 1, 16)
    oracle.set_threads(threads)
    model = oracle.Model(kind, weights(kind, size), size)
    one = (1,) + tuple(shape[1:])
    x = inputs(kind, one)
    model.forward(x)  # warm-up
    runs, t0 = 0, time.perf_counter()
    while True:
        model.forward(x)
        runs += 1
        el = time.perf_counter() - t0
        if el >= budget_s or runs >= 30:
            break
    unit = "images/s" if kind == "det" else "lines/s"
    return {"value": round(runs * one[0] / el, 3), "unit": unit, "cores": threads, "kind": "port",
            "sample": f"{runs} single-image passes of the {size} {'detector' if kind == 'det' else 'recognizer'} "
                      f"at {one}, C++ restatement of the reference CPU path (fp32, OpenMP)"}


def also(gpu, warmup, steps):
    out = {}
    configs = [
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
    for kind, size, shape, precision, *mode in configs:
        greedy = mode == ["greedy"]
        key = f"{size}_{kind}_{shape[0]}x{shape[2]}x{shape[3]}_{precision}" + ("_greedy" if greedy else "")
        try:
            m = load(gpu, kind, size, shape, precision, greedy)
            x = inputs(kind, shape)
            ms = throughput(m, x, warmup, steps)
            m.close()
            unit = "images/s" if kind == "det" else "lines/s"
            out[key] = {"value": round(shape[0] * steps / (ms / 1e3), 2), "unit": unit,
                        "ms_per_step": round(ms / steps, 4)}
        except Exception as e:  # report, keep going
            out[key] = {"error": str(e)}
    return out


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-extra", action="store_true", help="skip the other configurations")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a known-size copy kernel (for rocprofv3 counter scaling)")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: the detector/recognizer path has no multi-GPU form in this build "
              "(independent images shard across GPUs without communication); run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    kind, size, shape = "det", "medium", (8, 3, 416, 736)
    gpu = ppocr_hip.Gpu(0)
    model = load(gpu, kind, size, shape)
    x = inputs(kind, shape)
    total_ms = throughput(model, x, args.warmup, args.steps)
    ms_per_step = total_ms / args.steps
    value = shape[0] * args.steps / (total_ms / 1e3)
    stats = model.profile(x, runs=max(3, min(args.steps, 10)))
    roof = roofline(stats)
    model.close()

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "images/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
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
        "kernels": kernel_table(stats),
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(kind, size, shape)
    if not args.no_extra:
        line["also"] = also(gpu, args.warmup, max(5, args.steps // 2))
        line["pipeline"] = pipeline(gpu)
    gpu.close()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
