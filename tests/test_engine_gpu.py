"""End-to-end OCR engine (``OcrEngine::recognize``, src/ocr.rs:497-600) on
the device, checked stage by stage against the oracle.

The seeded detector gives a noise-like probability map, so a raised binary
threshold yields hundreds of small text regions: enough to exercise the
aspect-ratio ordering, batches of six, per-batch canvas widths and the
shape-keyed recognizer cache with eviction.  Checks:
* detection: the engine's lines are the device postprocess of the engine's
  own detector map, and that postprocess agrees with the oracle's
  ``extract_detections`` on the same map (bars of the postprocess tests);
* recognition: the oracle recognises the engine's polygons (same plans,
  oracle preprocessing, oracle recognizer, oracle greedy CTC) and gets the
  same text, with scores within 1e-3.
"""

import numpy as np
import pytest

import oracle
import ppocr_hip
import seeded
from helpers import model_path, quad_corners, synthetic_dictionary

pytestmark = pytest.mark.gpu

BATCH = 6  # RECOGNIZER_BATCH_SIZE, src/ocr.rs:22


@pytest.fixture(scope="module")
def gpu():
    g = ppocr_hip.Gpu(0)
    yield g
    g.close()


def aspect(q):
    w = max(np.linalg.norm(q[1] - q[0]), np.linalg.norm(q[2] - q[3]))
    h = max(np.linalg.norm(q[3] - q[0]), np.linalg.norm(q[2] - q[1]))
    return np.float32(w) / max(np.float32(h), np.float32(1.1920929e-7))


def oracle_recognize(img, polygons, dictionary):
    """recognize_with's recognition half (src/ocr.rs:541-571) on the oracle."""
    rec = oracle.Model("rec", model_path("rec", "tiny"), "tiny")
    order = sorted(range(len(polygons)), key=lambda i: aspect(polygons[i]))
    out = [None] * len(polygons)
    for s in range(0, len(order), BATCH):
        idx = order[s:s + BATCH]
        quads = np.stack([polygons[i] for i in idx])
        width = ppocr_hip.recognizer_batch_width(quads)
        content = [ppocr_hip.recognition_input_plan(q, width) for q in quads]
        x = np.stack([oracle.preprocess(img, q, width, 48, c, False) for q, c in zip(quads, content)])
        probs = rec.forward(x)
        for k, i in enumerate(idx):
            tokens, score = oracle.ctc_greedy_decode(probs[k], len(dictionary), content[k], width)
            srt = np.sort(probs[k], axis=-1)
            gap = float(np.min(srt[:, -1] - srt[:, -2]))  # smallest top-2 margin of the item
            out[i] = ("".join(dictionary[c - 1] for c in tokens), score, gap)
    return out


@pytest.mark.parametrize("greedy", [True, False])
def test_engine_matches_oracle_stage_by_stage(gpu, greedy):
    img = seeded.seeded_rgb(540, 960, 23, pattern="blocks")
    dictionary = synthetic_dictionary(6906)
    opts = dict(binary_threshold=0.62, box_threshold=0.0, min_area=3)
    engine = ppocr_hip.OcrEngine.load(gpu, model_path("det", "tiny"), model_path("rec", "tiny"), dictionary,
                                      greedy=greedy, **opts)
    try:
        result = engine.recognize(img)
    finally:
        engine.close()
    assert result.source_size == (960, 540)
    iw, ih = ppocr_hip.detector_input_plan(960, 540, 736)
    assert result.detector_input_size == (iw, ih)
    lines = result.lines
    assert len(lines) > 2 * BATCH

    # Detection stage.
    det = ppocr_hip.Detector.load(gpu, model_path("det", "tiny"), "tiny", (1, 3, ih, iw))
    image = gpu.upload_rgb(img)
    corners = quad_corners(0, 0, 960, 540)[None]
    try:
        prob = det.forward_image(image, corners).array()[0, 0]
        (dets,) = det.detect_image(image, corners, [(960, 540, iw, ih)], **opts)
    finally:
        image.close()
        det.close()
    assert len(dets) == len(lines)
    for d, ln in zip(dets, lines):
        assert np.abs(d.polygon - ln.polygon).max() <= 1e-3
        assert abs(d.score - ln.detection_score) <= 1e-6
    polys, scores, _ = oracle.extract_detections(prob, (960, 540, iw, ih), **opts)
    assert len(scores) == len(lines)
    assert np.allclose(np.sort(scores), np.sort([ln.detection_score for ln in lines]), atol=1e-6)

    # Recognition stage on the engine's own polygons.
    want = oracle_recognize(img, [ln.polygon for ln in lines], dictionary)
    # A text may differ only where some time step is a near-tie (top-2 gap
    # under 1e-4, the per-step parity bar).
    mismatched = [i for i, ln in enumerate(lines) if ln.text != want[i][0] and want[i][2] > 1e-4]
    assert not mismatched, f"{len(mismatched)} of {len(lines)} texts differ, first {mismatched[:5]}"
    err = max(abs(ln.recognition_score - w[1]) for ln, w in zip(lines, want))
    assert err <= 1e-3, err
    print(f"engine (greedy={greedy}): {len(lines)} lines, {sum(1 for ln in lines if ln.text)} non-empty")


def test_engine_default_options_and_image_sizes(gpu):
    # Three image sizes: three detector shapes, so the two-entry detector
    # cache evicts; repeated input gives identical output.
    dictionary = synthetic_dictionary(6906)
    engine = ppocr_hip.OcrEngine.load(gpu, model_path("det", "tiny"), model_path("rec", "tiny"), dictionary)
    try:
        results = []
        for h, w, seed in [(300, 500, 35), (540, 960, 23), (200, 200, 4), (300, 500, 35)]:
            img = seeded.seeded_rgb(h, w, seed, pattern="blocks")
            r = engine.recognize(img)
            assert r.source_size == (w, h)
            for ln in r.lines:
                assert np.all(ln.polygon[:, 0] >= 0) and np.all(ln.polygon[:, 0] <= w)
                assert np.all(ln.polygon[:, 1] >= 0) and np.all(ln.polygon[:, 1] <= h)
            results.append(r)
        a, b = results[0], results[-1]
        assert [ln.text for ln in a.lines] == [ln.text for ln in b.lines]
        assert all(np.abs(x.polygon - y.polygon).max() <= 1e-3 for x, y in zip(a.lines, b.lines))
    finally:
        engine.close()


def test_engine_page_without_detections(gpu):
    # A minimum component area no component reaches: the detector runs, the
    # postprocess keeps nothing, the recognizer gets an empty batch; the page
    # has no lines and still reports its sizes (src/ocr.rs:497-600 with an
    # empty detection list).  A blank page then runs through the same engine.
    dictionary = synthetic_dictionary(6906)
    engine = ppocr_hip.OcrEngine.load(gpu, model_path("det", "tiny"), model_path("rec", "tiny"), dictionary,
                                      min_area=10 ** 9)
    try:
        r = engine.recognize(seeded.seeded_rgb(240, 320, 3, pattern="blocks"))
        assert r.source_size == (320, 240)
        assert r.lines == []
        blank = engine.recognize(np.full((240, 320, 3), 255, np.uint8))
        assert blank.source_size == (320, 240) and blank.lines == []
    finally:
        engine.close()


def test_engine_rejects_mismatched_dictionary(gpu):
    with pytest.raises(ppocr_hip.GpuError) as e:
        ppocr_hip.OcrEngine.load(gpu, model_path("det", "tiny"), model_path("rec", "tiny"), ["a", "b"])
    assert e.value.kind == "InvalidInput"
    with pytest.raises(ppocr_hip.GpuError):
        ppocr_hip.OcrEngine.load(gpu, model_path("det", "tiny"), model_path("rec", "tiny"),
                                 synthetic_dictionary(6906), unclip_ratio=0.0)
