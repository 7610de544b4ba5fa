"""ppocr-gpu-bench, the benchmark CLI over the C ABI: the flag contract,
errors and report of the reference's `ppocr-gpu-bench`
(src/bin/ppocr-gpu-bench.rs:45-88, src/bin/benchmark.rs).

CPU tests cover argument handling and the checks the reference makes before
it opens a device (src/bin/benchmark.rs:60-79); GPU tests run the binary on
seeded tiny models and check the report, the dump and input files and the
reference comparison."""

import math
import pathlib
import re
import subprocess

import numpy as np
import pytest

from helpers import argmax_last, model_path

ROOT = pathlib.Path(__file__).resolve().parents[1]
CLI = ROOT / "ppocr-rs_amd" / "ppocr-gpu-bench"

pytestmark = pytest.mark.skipif(not CLI.exists(), reason="ppocr-gpu-bench not built (make -C ppocr-rs_amd)")


def run(*args, timeout=120):
    p = subprocess.run([str(CLI), *map(str, args)], capture_output=True, text=True, timeout=timeout)
    return p.returncode, p.stdout, p.stderr


def report(stdout):
    out = {}
    for line in stdout.splitlines():
        k, _, v = line.partition(": ")
        out[k] = v
    return out


def deterministic_input(length):
    """The LCG input of src/bin/benchmark.rs:126-134, in numpy float32."""
    state = 0x243F6A88
    top = np.empty(length, dtype=np.uint32)
    for i in range(length):
        state = (state * 1_664_525 + 1_013_904_223) & 0xFFFFFFFF
        top[i] = state >> 8
    unit = top.astype(np.float32) / np.float32(0x00FFFFFF)
    return unit * np.float32(2.0) - np.float32(1.0)


SCI = re.compile(r"^-?\d\.\d{9}e-?\d+$")


def rust_sci9(x):
    mant, exp = f"{x:.9e}".split("e")
    return f"{mant}e{int(exp)}"


# --- argument handling (no device) ---


def test_usage_errors_exit_with_status_2():
    rc, _, err = run()
    assert rc == 2 and "--kind" in err
    rc, _, err = run("--kind", "cls")
    assert rc == 2 and "invalid value 'cls'" in err
    rc, _, err = run("--kind", "det", "--offline", "--verify-models")
    assert rc == 2 and "cannot be used with" in err
    rc, _, err = run("--kind", "det", "--runs")
    assert rc == 2 and "a value is required" in err
    rc, _, err = run("--kind", "det", "--bogus", "1")
    assert rc == 2 and "unexpected argument" in err


def test_help_lists_the_reference_flags():
    rc, out, _ = run("--help")
    assert rc == 0
    for flag in ("--kind", "--model-size", "--model", "--model-dir", "--offline", "--verify-models", "--height",
                 "--width", "--input", "--reference", "--dump", "--warmup", "--runs"):
        assert flag in out


def test_checks_before_any_device_work(tmp_path):
    rc, _, err = run("--kind", "det", "--runs", "0")
    assert rc == 1 and err.strip() == "Error: --runs must be positive"
    rc, _, err = run("--kind", "rec", "--height", "0")
    assert rc == 1 and err.strip() == "Error: --height must be positive"
    rc, _, err = run("--kind", "rec", "--width=0")
    assert rc == 1 and err.strip() == "Error: --width must be positive"
    bad = tmp_path / "short.f32"
    bad.write_bytes(b"\0" * 8)
    rc, _, err = run("--kind", "det", "--height", "64", "--width", "96", "--input", bad)
    assert rc == 1 and "must contain 18432 F32 values, found 8 bytes" in err
    rc, _, err = run("--kind", "det", "--model-dir", tmp_path)
    assert rc == 1 and f"tiny-det is missing in {tmp_path}/tiny-det" in err
    rc, _, err = run("--kind", "rec", "--model-size", "small", "--verify-models")
    assert rc == 1 and "pinned model catalog" in err


def test_model_cache_layout_is_size_then_kind(tmp_path, monkeypatch):
    # <dir>/<size>-<kind>/model.safetensors (src/models.rs:325-344); an
    # empty file there gets past resolution and fails in the loader.
    d = tmp_path / "medium-rec"
    d.mkdir()
    (d / "model.safetensors").write_bytes(b"")
    monkeypatch.setenv("PPOCR_MODEL_DIR", str(tmp_path))
    rc, _, err = run("--kind", "rec", "--model-size", "medium", "--runs", "1")
    assert rc == 1 and "is missing in" not in err


# --- on the device ---


@pytest.mark.gpu
def test_detector_report_dump_input_and_reference(tmp_path):
    import oracle

    weights = model_path("det", "tiny")
    a, b = tmp_path / "a.f32", tmp_path / "b.f32"
    rc, out, err = run("--kind", "det", "--model", weights, "--height", "64", "--width", "96", "--warmup", "1",
                       "--runs", "5", "--dump", a)
    assert rc == 0, err
    r = report(out)
    assert list(r)[:15] == ["backend", "kind", "model", "input_shape", "output_shape", "output_min", "output_max",
                            "output_sum", "warmup", "runs", "average_ms", "p50_ms", "p90_ms", "p95_ms", "throughput"]
    assert r["kind"] == "det" and r["model"] == str(weights)
    assert r["input_shape"] == "[1, 3, 64, 96]" and r["output_shape"] == "[1, 1, 64, 96]"
    assert r["warmup"] == "1" and r["runs"] == "5" and r["dump"] == str(a)
    got = np.fromfile(a, dtype="<f4")
    assert got.size == 64 * 96 and np.all(np.isfinite(got))
    for key in ("output_min", "output_max", "output_sum"):
        assert SCI.match(r[key]), r[key]
    assert r["output_min"] == rust_sci9(float(got.min()))
    assert r["output_max"] == rust_sci9(float(got.max()))
    assert r["output_sum"] == rust_sci9(float(np.cumsum(got.astype(np.float64))[-1]))
    avg, p50, p90, p95 = (float(r[k]) for k in ("average_ms", "p50_ms", "p90_ms", "p95_ms"))
    assert 0 < p50 <= p90 <= p95
    assert math.isclose(float(r["throughput"]), 1000.0 / avg, rel_tol=0.01)

    # The generated input is the reference's LCG: the same bytes through
    # --input give the same output bit for bit.
    x = deterministic_input(3 * 64 * 96)
    inp = tmp_path / "x.f32"
    x.astype("<f4").tofile(inp)
    rc, out, err = run("--kind", "det", "--model", weights, "--height", "64", "--width", "96", "--warmup", "0",
                       "--runs", "1", "--input", inp, "--dump", b, "--reference", a)
    assert rc == 0, err
    assert np.array_equal(np.fromfile(b, dtype="<f4"), got)
    r = report(out)
    assert r["reference_max_abs"] == "0.000000000e0"
    assert r["reference_mean_abs"] == "0.000000000e0"
    assert r["reference_threshold_0.5_mismatches"] == "0"

    # And the output is the oracle's detector on that input.
    want = oracle.Model("det", weights, "tiny").forward(x.reshape(1, 3, 64, 96)).reshape(-1)
    assert float(np.max(np.abs(got - want))) <= 1e-3

    # reference_threshold_0.5_mismatches counts the pixels whose side of 0.5
    # differs; max/mean abs as src/bin/benchmark.rs:250-258.
    ref = got.copy()
    flip = np.argsort(np.abs(got - 0.5))[:3]
    ref[flip] = np.where(got[flip] >= 0.5, np.float32(0.25), np.float32(0.75))
    ref.astype("<f4").tofile(b)
    rc, out, err = run("--kind", "det", "--model", weights, "--height", "64", "--width", "96", "--warmup", "0",
                       "--runs", "1", "--reference", b)
    assert rc == 0, err
    r = report(out)
    d = np.abs(got - ref)
    assert r["reference_threshold_0.5_mismatches"] == "3"
    assert r["reference_max_abs"] == rust_sci9(float(d.max()))
    assert r["reference_mean_abs"] == rust_sci9(float(np.cumsum(d.astype(np.float64))[-1] / d.size))


@pytest.mark.gpu
def test_recognizer_argmax_mismatches_and_batch(tmp_path):
    weights = model_path("rec", "tiny")
    a = tmp_path / "a.f32"
    rc, out, err = run("--kind", "rec", "--model", weights, "--width", "64", "--batch", "2", "--warmup", "1",
                       "--runs", "3", "--dump", a)
    assert rc == 0, err
    r = report(out)
    assert r["input_shape"] == "[2, 3, 48, 64]"
    shape = [int(v) for v in r["output_shape"].strip("[]").split(", ")]
    assert shape[0] == 2 and shape[2] == 6906
    assert float(r["items_per_second"]) > 0
    probs = np.fromfile(a, dtype="<f4").reshape(-1, shape[2])
    # Move the maximum of two time steps to another class.
    ref = probs.copy()
    top = argmax_last(ref)
    for row in (0, len(ref) - 1):
        other = (top[row] + 1) % shape[2]
        ref[row, other] = ref[row, top[row]] + np.float32(0.5)
    ref.astype("<f4").tofile(tmp_path / "ref.f32")
    rc, out, err = run("--kind", "rec", "--model", weights, "--width", "64", "--batch", "2", "--warmup", "0",
                       "--runs", "1", "--reference", tmp_path / "ref.f32")
    assert rc == 0, err
    assert report(out)["reference_argmax_mismatches"] == "2"
