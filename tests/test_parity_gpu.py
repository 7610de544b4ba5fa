"""Parity of the HIP backend against the CPU oracle on identical seeded
inputs and weights (run on an MI355X: ``pytest -m gpu``).

Bars:
* detector probability maps: max |diff| <= 1e-3 (fp32 accumulate), and the
  DB binarisation at 0.2 / 0.5 identical outside a 1e-5 ambiguity band;
* recognizer softmax probabilities: max |diff| <= 1e-3, argmax identical
  where the top-2 gap exceeds 1e-4, greedy-CTC strings identical;
* preprocessing: bit-exact (integer rounding of the bilinear sample).
"""

import numpy as np
import pytest

import oracle
import ppocr_hip
import seeded
from helpers import (argmax_last, band_mismatches, ctc_greedy, edit_distance, model_path, quad_corners,
                     synthetic_dictionary)

pytestmark = pytest.mark.gpu

DET_TOL = 1e-3
REC_TOL = 1e-3


@pytest.fixture(scope="module")
def gpu():
    g = ppocr_hip.Gpu(0)
    yield g
    g.close()


_oracles = {}


def oracle_model(kind, size):
    key = (kind, size)
    if key not in _oracles:
        _oracles[key] = oracle.Model(kind, model_path(kind, size), size)
    return _oracles[key]


def check_detector(actual, expected):
    assert actual.shape == expected.shape
    err = float(np.max(np.abs(actual - expected)))
    assert err <= DET_TOL, f"max abs diff {err}"
    for thr in (0.2, 0.5):
        mism, band = band_mismatches(actual, expected, thr)
        assert mism == 0, f"{mism} mask mismatches at {thr} (band {band})"
    return err


def check_recognizer(actual, expected):
    assert actual.shape == expected.shape
    err = float(np.max(np.abs(actual - expected)))
    assert err <= REC_TOL, f"max abs diff {err}"
    srt = np.sort(expected, axis=-1)
    clear = (srt[..., -1] - srt[..., -2]) > 1e-4
    am_a, am_e = argmax_last(actual), argmax_last(expected)
    assert np.all(am_a[clear] == am_e[clear])
    return err


@pytest.mark.parametrize("size,shape,seed,pattern", [
    ("tiny", (1, 3, 416, 736), 7, "uniform"),
    ("tiny", (2, 3, 64, 96), 3, "uniform"),
    ("tiny", (1, 3, 832, 1472), 5, "blocks"),
    ("small", (1, 3, 416, 736), 7, "uniform"),
    ("small", (8, 3, 416, 736), 11, "uniform"),
    ("medium", (1, 3, 416, 736), 7, "uniform"),
    ("medium", (2, 3, 128, 160), 9, "uniform"),
    ("medium", (8, 3, 416, 736), 13, "uniform"),  # the throughput benchmark's batch (split-K choices differ)
])
def test_detector_matches_oracle(gpu, size, shape, seed, pattern):
    x = seeded.seeded_batch(shape[0], shape[2], shape[3], seed, detector=True, pattern=pattern)
    det = ppocr_hip.Detector.load(gpu, model_path("det", size), size, shape)
    try:
        out = det.forward(x)
        assert out.shape == [shape[0], 1, shape[2], shape[3]]
        expected = oracle_model("det", size).forward(x)
        err = check_detector(out.array(), expected)
        print(f"det {size} {shape}: max abs {err:.2e}")
    finally:
        det.close()


@pytest.mark.parametrize("size,batch,width", [
    ("tiny", 4, 320),
    ("tiny", 64, 320),
    ("tiny", 3, 100),
    ("small", 4, 320),
    ("medium", 4, 320),
    ("medium", 2, 648),
    ("medium", 256, 320),  # the long-batch benchmark shape
])
def test_recognizer_matches_oracle(gpu, size, batch, width):
    x = seeded.seeded_batch(batch, 48, width, 100 + batch, detector=False)
    shape = (batch, 3, 48, width)
    rec = ppocr_hip.Recognizer.load(gpu, model_path("rec", size), size, shape)
    try:
        out = rec.forward(x).array()
        expected = oracle_model("rec", size).forward(x)
        err = check_recognizer(out, expected)
        dictionary = synthetic_dictionary(expected.shape[-1])
        for i in range(batch):
            assert ctc_greedy(out[i], dictionary, width, width)[0] == ctc_greedy(expected[i], dictionary, width,
                                                                               width)[0]
        print(f"rec {size} {shape}: max abs {err:.2e}")
    finally:
        rec.close()


# bf16 storage (activations and matrix-core weights in bf16, fp32 accumulate
# and epilogues) against the fp32 oracle.  The yardstick is the oracle's bf16
# emulation: the same network with the values a bf16 plan rounds to bf16
# rounded at the same points, and the same weights taken in bf16 (the
# rounding function and the list of rounding points are pinned on the CPU,
# tests/test_bf16_emulation.py).  E = |emulation - fp32| on the same input
# is what bf16 storage alone costs.  The seeded networks amplify a rounding
# difference by ~10x per few layers, so a rounding that the device's fp32
# summation order flips and the emulation's does not moves an output by as
# much as E itself (measured: reversing the emulation's summation order
# moves the tiny detector's map by 0.053 against E = 0.080); the bars are
# therefore statistical in E, not bit-level:
#   max and mean |device - fp32| <= F x (max, mean) of E, plus 1e-3 / 1e-4
#     (detector / recognizer) for the fp32 kernels' own rounding, F = 2;
#   detector: the DB masks at 0.2 and 0.5 identical wherever the fp32 value
#     is further than that max bound from the threshold, and over the whole
#     map the device's mask pixels that differ from fp32's at most 1.5x the
#     emulation's (plus 0.05 % of the pixels);
#   recognizer: in logit space (log p of the fp32 top-2 classes), G = F x
#     the largest change the emulation makes to any step's top-2 logit gap;
#     the argmax is identical on every step whose fp32 logit gap exceeds G
#     (at least half the steps), and the greedy CTC string is identical on
#     every line all of whose steps do; over all steps, the device's argmax
#     disagreements with fp32 are at most 1.5x the emulation's (plus 10), and
#     over all lines the edit distance of the device's CTC strings to fp32's
#     at most 1.5x the emulation's (plus 5 tokens).  (Line-level string
#     equality on every line cannot be asked of a random-weight network in
#     bf16: its encoder features carry ~1.6 % RMS noise from bf16 storage,
#     and the seeded recognizers whose every step clears that noise are the
#     collapsed ones that emit one or two classes.)
BF16_F = 2.0


def bf16_emulation(kind, size, x):
    oracle.set_bf16(True)
    try:
        return oracle.Model(kind, model_path(kind, size), size).forward(x)
    finally:
        oracle.set_bf16(False)


@pytest.mark.parametrize("kind,size,shape", [
    ("det", "tiny", (1, 3, 416, 736)),
    ("det", "small", (2, 3, 416, 736)),
    ("det", "medium", (1, 3, 416, 736)),
    ("det", "medium", (8, 3, 416, 736)),
    ("rec", "tiny", (16, 3, 48, 320)),
    ("rec", "small", (16, 3, 48, 320)),
    ("rec", "medium", (16, 3, 48, 320)),
    ("rec", "medium", (256, 3, 48, 320)),
])
def test_bf16_storage_within_derived_tolerance(gpu, kind, size, shape):
    x = seeded.seeded_batch(shape[0], shape[2], shape[3], 31, detector=(kind == "det"))
    cls = ppocr_hip.Detector if kind == "det" else ppocr_hip.Recognizer
    m = cls.load(gpu, model_path(kind, size), size, shape, precision="bf16")
    try:
        y = m.forward(x).array()
    finally:
        m.close()
    ref = oracle_model(kind, size).forward(x)
    emu = bf16_emulation(kind, size, x)
    d, e = np.abs(y - ref), np.abs(emu - ref)
    floor = 1e-3 if kind == "det" else 1e-4
    print(f"bf16 {kind} {size} {shape}: device max {d.max():.3e} mean {d.mean():.3e}; "
          f"emulation max {e.max():.3e} mean {e.mean():.3e}")
    assert d.max() <= BF16_F * e.max() + floor, (d.max(), e.max())
    assert d.mean() <= BF16_F * e.mean() + floor / 10, (d.mean(), e.mean())
    if kind == "det":
        band = BF16_F * e.max() + floor
        for thr in (0.2, 0.5):
            far = np.abs(ref - thr) > band
            assert np.all((y >= thr)[far] == (ref >= thr)[far]), f"mask differs outside the {band:.3f} band at {thr}"
            assert far.mean() > 0.5  # the check covers most of the map
            mis_dev = int(np.count_nonzero((y >= thr) != (ref >= thr)))
            mis_emu = int(np.count_nonzero((emu >= thr) != (ref >= thr)))
            print(f"  mask at {thr}: device differs from fp32 on {mis_dev} pixels, emulation on {mis_emu}")
            assert mis_dev <= 1.5 * mis_emu + 5e-4 * ref.size, (thr, mis_dev, mis_emu)
    else:
        top = np.argsort(ref, axis=-1)[..., -2:]

        def gap(p):
            lp = np.log(np.maximum(p, 1e-30))
            return (np.take_along_axis(lp, top[..., 1:], -1) - np.take_along_axis(lp, top[..., :1], -1))[..., 0]

        g_ref = gap(ref)
        bound = BF16_F * np.abs(gap(emu) - g_ref).max()
        confident = g_ref > bound
        print(f"  logit-gap bound {bound:.3f}: {confident.mean():.1%} of steps confident")
        assert confident.mean() >= 0.5
        assert np.all(argmax_last(y)[confident] == argmax_last(ref)[confident])
        am_ref = argmax_last(ref)
        dis_dev = int(np.count_nonzero(argmax_last(y) != am_ref))
        dis_emu = int(np.count_nonzero(argmax_last(emu) != am_ref))
        print(f"  step argmax differs from fp32: device {dis_dev}, emulation {dis_emu} of {am_ref.size}")
        assert dis_dev <= 1.5 * dis_emu + 10, (dis_dev, dis_emu)
        dictionary = synthetic_dictionary(ref.shape[-1])
        width = shape[3]
        lines = [i for i in range(shape[0]) if confident[i].all()]
        print(f"  {len(lines)} of {shape[0]} lines fully confident")
        tokens = lambda p: oracle.ctc_greedy_decode(p, len(dictionary), width, width)[0]  # noqa: E731
        for i in lines:
            assert ctc_greedy(y[i], dictionary, width, width)[0] == ctc_greedy(ref[i], dictionary, width, width)[0]
        want = [tokens(ref[i]) for i in range(shape[0])]
        d_dev = sum(edit_distance(tokens(y[i]), want[i]) for i in range(shape[0]))
        d_emu = sum(edit_distance(tokens(emu[i]), want[i]) for i in range(shape[0]))
        print(f"  CTC edit distance to fp32 over {shape[0]} lines ({sum(map(len, want))} tokens): device {d_dev}, "
              f"emulation {d_emu}")
        assert d_dev <= 1.5 * d_emu + 5, (d_dev, d_emu)


def test_preprocess_is_bit_exact(gpu):
    rng = np.random.default_rng(5)
    img = rng.integers(0, 256, size=(97, 211, 3), dtype=np.uint8)
    image = gpu.upload_rgb(img)
    cases = [
        (quad_corners(0, 0, 211, 97), 160, 64, 160, True),
        (np.array([[2.25, 1.75], [190.5, 3.0], [182.75, 90.0], [1.0, 85.5]], np.float32), 320, 48, 201, False),
        (np.array([[10.0, 80.0], [200.0, 5.0], [205.0, 30.0], [12.0, 96.0]], np.float32), 128, 48, 128, False),
    ]
    for corners, cw, ch, content, det in cases:
        got = gpu.preprocess(image, corners, cw, ch, content, det)
        want = oracle.preprocess(img, corners, cw, ch, content, det)
        assert np.array_equal(got, want), f"max diff {np.max(np.abs(got - want))}"
    image.close()


def test_detector_forward_image_matches_host_preprocess(gpu):
    img = seeded.seeded_rgb(540, 960, 21)
    h, w = 416, 736
    det = ppocr_hip.Detector.load(gpu, model_path("det", "tiny"), "tiny", (1, 3, h, w))
    image = gpu.upload_rgb(img)
    try:
        corners = quad_corners(0, 0, 960, 540)
        out = det.forward_image(image, corners[None]).array()
        x = oracle.preprocess(img, corners, w, h, w, True)[None]
        expected = oracle_model("det", "tiny").forward(x)
        check_detector(out, expected)
    finally:
        image.close()
        det.close()


@pytest.mark.parametrize("precision", ["f32", "bf16"])
@pytest.mark.parametrize("kind", ["det", "rec"])
def test_forward_image_equals_forward_of_device_preprocess(gpu, kind, precision):
    """Device preprocessing writes the model input (NHWC4, activation type)
    itself and the plan skips its input conversion: the result must be the
    forward pass of the preprocessed planes, bit for bit."""
    img = seeded.seeded_rgb(300, 500, 41, pattern="blocks")
    quads = np.stack([quad_corners(0, 0, 500, 300), np.array([[40, 30], [420, 50], [410, 260], [30, 240]], np.float32)])
    if kind == "det":
        h, w, widths = 64, 96, None
        model = ppocr_hip.Detector.load(gpu, model_path("det", "tiny"), "tiny", (2, 3, h, w), precision=precision)
    else:
        h, w, widths = 48, 128, [128, 72]
        model = ppocr_hip.Recognizer.load(gpu, model_path("rec", "tiny"), "tiny", (2, 3, h, w), precision=precision)
    image = gpu.upload_rgb(img)
    try:
        got = model.forward_image(image, quads, widths).array()
        x = np.stack([gpu.preprocess(image, q, w, h, None if widths is None else widths[i], kind == "det")
                      for i, q in enumerate(quads)])
        want = model.forward(x).array()
        assert np.array_equal(got, want)
    finally:
        image.close()
        model.close()


def test_recognizer_forward_image_batched_crops(gpu):
    img = seeded.seeded_rgb(300, 500, 33, pattern="blocks")
    quads = np.stack([quad_corners(10, 20, 210, 60), quad_corners(100, 100, 180, 120),
                      np.array([[300, 200], [480, 210], [478, 250], [298, 240]], np.float32)])
    widths = [240, 192, 216]
    n, width = len(quads), 320
    rec = ppocr_hip.Recognizer.load(gpu, model_path("rec", "tiny"), "tiny", (n, 3, 48, width))
    image = gpu.upload_rgb(img)
    try:
        out = rec.forward_image(image, quads, widths).array()
        x = np.stack([oracle.preprocess(img, q, width, 48, cw, False) for q, cw in zip(quads, widths)])
        expected = oracle_model("rec", "tiny").forward(x)
        check_recognizer(out, expected)
    finally:
        image.close()
        rec.close()


def test_recognizers_share_device_weights(gpu):
    path = model_path("rec", "tiny")
    a = ppocr_hip.Recognizer.load(gpu, path, "tiny", (2, 3, 48, 320))
    b = ppocr_hip.Recognizer.load(gpu, path, "tiny", (1, 3, 48, 160), share_weights=a)
    try:
        x = seeded.seeded_batch(1, 48, 160, 77, detector=False)
        check_recognizer(b.forward(x).array(), oracle_model("rec", "tiny").forward(x))
        assert b.memory_report()["weight_bytes"] == a.memory_report()["weight_bytes"]
    finally:
        b.close()
        a.close()


def test_invalid_inputs_are_rejected(gpu):
    path = model_path("det", "tiny")
    with pytest.raises(ppocr_hip.GpuError) as e:
        ppocr_hip.Detector.load(gpu, path, "tiny", (1, 3, 100, 96))
    assert e.value.kind == "InvalidInput"
    with pytest.raises(ppocr_hip.GpuError) as e:
        ppocr_hip.Detector.load(gpu, path, "medium", (1, 3, 64, 64))
    assert e.value.kind == "InvalidModel"
    with pytest.raises(ppocr_hip.GpuError) as e:
        ppocr_hip.Detector.load(gpu, "/nonexistent/weights.safetensors", "tiny", (1, 3, 64, 64))
    assert e.value.kind == "ReadFile"
    det = ppocr_hip.Detector.load(gpu, path, "tiny", (1, 3, 64, 64))
    try:
        with pytest.raises(ppocr_hip.GpuError) as e:
            det.forward(np.zeros((1, 3, 64, 32), np.float32))
        assert e.value.kind == "InvalidInput"
        bad = np.zeros((1, 3, 64, 64), np.float32)
        bad[0, 1, 5, 5] = np.nan
        with pytest.raises(ppocr_hip.GpuError) as e:
            det.forward(bad)
        assert e.value.kind == "InvalidInput"
        good = seeded.seeded_batch(1, 64, 64, 1)
        check_detector(det.forward(good).array(), oracle_model("det", "tiny").forward(good))
    finally:
        det.close()


def test_benchmark_and_profile_report(gpu):
    x = seeded.seeded_batch(1, 416, 736, 7)
    det = ppocr_hip.Detector.load(gpu, model_path("det", "tiny"), "tiny", x.shape)
    try:
        samples = det.benchmark(x, warmup=2, runs=5)
        assert len(samples) == 5 and all(s > 0 for s in samples)
        stats = det.profile(x, runs=3)
        assert stats and all(s["avg_ms"] >= 0 for s in stats)
        total = det.benchmark_stream(x, 2, 10)
        assert total > 0
        # The pass after profiling still matches the oracle (no stale state).
        check_detector(det.forward(x).array(), oracle_model("det", "tiny").forward(x))
    finally:
        det.close()


# Greedy recognizer: the classifier fused with per-step greedy CTC decoding
# (src/ocr.rs:800-853).  Bars: the step class equals the oracle's argmax
# (ties -> last) wherever the oracle's top-2 probability gap exceeds 1e-4,
# the step probability is within 1e-3 of the oracle's, and the decoded
# strings are identical.
def check_greedy(steps, expected, width, content_widths=None):
    n, t, v = expected.shape
    assert steps.shape == (n, t, 2)
    cls = steps[..., 0]
    assert np.all(cls == np.round(cls)) and cls.min() >= 0 and cls.max() < v
    srt = np.sort(expected, axis=-1)
    clear = (srt[..., -1] - srt[..., -2]) > 1e-4
    am = argmax_last(expected)
    assert np.all(cls.astype(np.int64)[clear] == am[clear])
    err = float(np.max(np.abs(steps[..., 1] - srt[..., -1])))
    assert err <= REC_TOL, f"probability max abs diff {err}"
    dictionary = synthetic_dictionary(v)
    for i in range(n):
        cw = width if content_widths is None else content_widths[i]
        got = ppocr_hip.ctc_greedy_decode(steps[i], dictionary, v, cw, width)
        want_text, want_score = ctc_greedy(expected[i], dictionary, cw, width)
        assert got.text == want_text
        assert abs(got.score - want_score) <= 1e-3
    return err


@pytest.mark.parametrize("size,batch,width", [
    ("tiny", 4, 320),
    ("tiny", 3, 100),
    ("small", 4, 320),
    ("medium", 4, 320),
    ("medium", 64, 320),
])
def test_greedy_recognizer_matches_oracle(gpu, size, batch, width):
    x = seeded.seeded_batch(batch, 48, width, 200 + batch, detector=False)
    shape = (batch, 3, 48, width)
    rec = ppocr_hip.Recognizer.load(gpu, model_path("rec", size), size, shape, greedy=True)
    try:
        steps = rec.forward(x).array()
    finally:
        rec.close()
    expected = oracle_model("rec", size).forward(x)
    err = check_greedy(steps, expected, width)
    print(f"greedy rec {size} {shape}: prob max abs {err:.2e}")


def test_greedy_recognizer_agrees_with_probability_output(gpu):
    # Same device arithmetic up to the classifier: the fused reduction must
    # reproduce the argmax and probability of the stored softmax rows.
    for precision in ("f32", "bf16"):
        shape = (16, 3, 48, 320)
        x = seeded.seeded_batch(16, 48, 320, 41, detector=False)
        path = model_path("rec", "medium")
        probs_model = ppocr_hip.Recognizer.load(gpu, path, "medium", shape, precision=precision)
        greedy = ppocr_hip.Recognizer.load(gpu, path, "medium", shape, precision=precision,
                                           share_weights=probs_model, greedy=True)
        try:
            probs = probs_model.forward(x).array()
            steps = greedy.forward(x).array()
            assert greedy.memory_report()["weight_bytes"] == probs_model.memory_report()["weight_bytes"]
        finally:
            greedy.close()
            probs_model.close()
        srt = np.sort(probs, axis=-1)
        clear = (srt[..., -1] - srt[..., -2]) > 1e-5
        assert np.all(steps[..., 0].astype(np.int64)[clear] == argmax_last(probs)[clear]), precision
        assert np.max(np.abs(steps[..., 1] - srt[..., -1])) <= 1e-5, precision


def test_greedy_recognizer_forward_image(gpu):
    img = seeded.seeded_rgb(300, 500, 35, pattern="blocks")
    quads = np.stack([quad_corners(10, 20, 210, 60), quad_corners(100, 100, 180, 120),
                      np.array([[300, 200], [480, 210], [478, 250], [298, 240]], np.float32)])
    width = ppocr_hip.recognizer_batch_width(quads)
    widths = [ppocr_hip.recognition_input_plan(q, width) for q in quads]
    n = len(quads)
    rec = ppocr_hip.Recognizer.load(gpu, model_path("rec", "tiny"), "tiny", (n, 3, 48, width), greedy=True)
    image = gpu.upload_rgb(img)
    try:
        steps = rec.forward_image(image, quads, widths).array()
    finally:
        image.close()
        rec.close()
    x = np.stack([oracle.preprocess(img, q, width, 48, cw, False) for q, cw in zip(quads, widths)])
    check_greedy(steps, oracle_model("rec", "tiny").forward(x), width, widths)
