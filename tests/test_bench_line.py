"""The benchmark's headline record: the last stdout line must stay short
enough that a tail of the output (the driver keeps about 8 KB) holds it
whole, and carry the fields of the bench contract.  CPU only: the record is
built from synthetic measurements shaped like a full run's."""

import importlib
import json
import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _bench():
    if str(ROOT) not in sys.path:
        sys.path.insert(0, str(ROOT))
    return importlib.import_module("bench")


def _fake_stats(n_kernels=120):
    names = [f"conv_gemm<64x64,1x1,variant{i % 17}>" for i in range(n_kernels)]
    return [{"kernel": n, "bound": "mfma" if i % 3 else "hbm", "avg_ms": 0.01 + 0.001 * i,
             "flops": 5.4e9, "bytes": 9.6e7} for i, n in enumerate(names)]


def _fake_config_record(bench, stats):
    return {"value": 123456.78, "unit": "lines/s", "ms_per_step": 1.2345,
            "roofline": bench.roofline(stats, "no_such_workload"), "pass": bench.pass_rates(stats, 4.77, "f32"),
            "kernels": bench.kernel_table(stats, 5)}


def test_headline_line_is_short_and_complete():
    bench = _bench()
    stats = _fake_stats()
    roof = bench.roofline(stats, "no_such_workload")
    extra = {}
    for kind, size, shape, precision, *mode in bench.ALSO_CONFIGS:
        extra[bench.config_key(kind, size, shape, precision, mode == ["greedy"])] = _fake_config_record(bench, stats)
    # Headroom: three more configurations than the bench measures today.
    for i in range(3):
        extra[f"small_rec_256x48x320_bf16_greedy_{i}"] = _fake_config_record(bench, stats)
    extra["broken_config"] = {"error": "x" * 5000}
    cpu = {"value": 1.03, "unit": "images/s", "cores": 4, "kind": "port", "sample": "s" * 300,
           "cpus": "os.cpu_count()=256, affinity=16, OMP_NUM_THREADS=16",
           "others": [{"workload": "tiny recognizer 1x3x48x320", "value": 98.1, "unit": "lines/s", "cores": 16}] * 4}
    line = bench.headline(1675.7, 20, 5, 4.7742, (8, 3, 416, 736), roof, bench.pass_rates(stats, 4.77, "f32"),
                          cpu, extra)
    assert "\n" not in line
    assert len(line.encode()) < 4096, len(line.encode())
    rec = json.loads(line)
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in rec, key
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in rec["roofline"], key
    for key in ("value", "unit", "cores", "kind", "sample"):
        assert key in rec["cpu_baseline"], key
    assert rec["config"]["workload"].startswith("PP-OCRv6 medium detector")
    assert all("kernels" not in v for v in rec["also"].values())


def test_detail_lines_are_json(capsys):
    bench = _bench()
    bench.emit("probe", {"a": [1, 2, 3]})
    out = capsys.readouterr().out.strip().splitlines()
    assert json.loads(out[-1]) == {"detail": "probe", "data": {"a": [1, 2, 3]}}


def test_roof_follows_arithmetic_intensity():
    """A matrix-core group is measured against the matrix peak only from the
    ridge point (peak FLOP/s / 8 TB/s) up, against HBM below it."""
    bench = _bench()

    def group(flops, nbytes, bound="mfma"):
        return {"ms": 0.05, "flops": flops, "bytes": nbytes, "launches": 1, "bound": bound}

    # fp32 ridge 157.3e12 / 8e12 = 19.66 FLOP/B; bf16 ridge 312.5 FLOP/B.
    assert bench.bound_of(group(6.4e9, 1.055e8), "f32") == "mfma"  # 60.7 FLOP/B
    assert bench.bound_of(group(1.9e9, 1.055e8), "f32") == "hbm"  # 18.0 FLOP/B
    assert bench.bound_of(group(6.4e9, 1.055e8), "bf16") == "hbm"
    assert bench.bound_of(group(1.3e11, 3.77e8), "bf16") == "mfma"  # 345 FLOP/B
    assert bench.bound_of(group(1e9, 1e8, "valu"), "f32") == "valu"  # 10 >= 9.83
    assert bench.bound_of(group(9e8, 1e8, "valu"), "f32") == "hbm"
    assert bench.bound_of(group(0.0, 1e8, "hbm"), "f32") == "hbm"
    # Below the ridge the fraction is bytes over the HBM peak, which equals
    # FLOPs over the attainable intensity x bandwidth.
    g = group(6.4e9, 1.055e8)
    achieved, peak, unit = bench.rate(g, "bf16")
    assert unit == "GB/s" and peak == bench.PEAK_HBM_GBS
    flops_rate = 6.4e9 / 0.05e-3
    attainable = 6.4e9 / 1.055e8 * bench.PEAK_HBM_GBS * 1e9
    assert abs(achieved / peak - flops_rate / attainable) < 1e-9
