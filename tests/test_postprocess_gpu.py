"""Device DB postprocess against the oracle's restatement of
``extract_detections`` (src/ocr.rs:723-790), on the same probability maps.

Bars: the same number of detections; every oracle detection matched by one
device detection with the same score (within 1e-6: the device sums in fp64
in another order) and, where the component's principal axis is determined
(oracle anisotropy > 1e-2), the same polygon within 1e-2 source pixels.  For
near-isotropic components the axis is decided by rounding noise in the
reference itself, so only the score and centre are compared.  The order is
the reference's positional order up to centres that tie within 1e-2.
"""

import numpy as np
import pytest

import oracle
import ppocr_hip
import seeded
from helpers import model_path, quad_corners

pytestmark = pytest.mark.gpu

POLY_TOL = 1e-2
SCORE_TOL = 1e-6


@pytest.fixture(scope="module")
def gpu():
    g = ppocr_hip.Gpu(0)
    yield g
    g.close()


def check(dets, values, transform, scale=1.0, **opts):
    polys, scores, aniso = oracle.extract_detections(values, transform, **opts)
    assert len(dets) == len(scores), (len(dets), len(scores))
    if not dets:
        return 0
    got_c = np.array([d.polygon.mean(0) for d in dets])
    want_c = polys.mean(1)
    used = set()
    for i in range(len(scores)):
        dist = np.abs(got_c - want_c[i]).max(1)
        dist[list(used)] = np.inf
        j = int(np.argmin(dist))
        used.add(j)
        assert dist[j] <= max(0.5, POLY_TOL) * scale, f"no device detection near oracle {i}"
        assert abs(dets[j].score - scores[i]) <= SCORE_TOL
        if aniso[i] > 1e-2:
            err = np.abs(dets[j].polygon - polys[i]).max()
            assert err <= POLY_TOL * scale, f"detection {i}: polygon off by {err}"
        if j != i:  # only a near-tie in the positional key may reorder
            assert abs(want_c[i, 1] - want_c[j, 1]) <= POLY_TOL * scale
    return len(dets)


def blob_map(rng, h, w, blobs=12):
    v = rng.random((h, w)).astype(np.float32) * 0.25
    for _ in range(blobs):
        y0, x0 = rng.integers(0, h - 3), rng.integers(0, w - 3)
        v[y0:y0 + rng.integers(1, 14), x0:x0 + rng.integers(1, 30)] = rng.uniform(0.3, 1.0)
    return v


def test_reference_literal(gpu):
    values = np.zeros((416, 736), np.float32)
    values[20:22, 10:14] = 0.9
    (dets,) = gpu.db_postprocess(values, [(736, 416, 736, 416)], min_area=4, unclip_ratio=1.0)
    assert len(dets) == 1
    assert abs(dets[0].score - 0.9) < 1e-6
    assert abs(dets[0].polygon[0, 0] - 10.0) < 1e-4


def test_empty_and_below_threshold_maps(gpu):
    # No pixel at the binary threshold (0.2): no components, no detections,
    # in a batch with a map that has one; a component whose mean score is
    # under the box threshold (0.4) is dropped.
    h, w = 64, 96
    zero = np.zeros((h, w), np.float32)
    under = np.full((h, w), 0.1999, np.float32)
    one = np.zeros((h, w), np.float32)
    one[10:20, 10:40] = 0.9
    weak = np.zeros((h, w), np.float32)
    weak[10:20, 10:40] = 0.39
    maps = np.stack([zero, under, one, weak])
    out = gpu.db_postprocess(maps, [(w, h, w, h)] * 4)
    assert [len(d) for d in out] == [0, 0, 1, 0]
    for i in range(4):
        check(out[i], maps[i], (w, h, w, h))


def test_component_touching_every_border(gpu):
    # A frame one pixel inside the map edge and a block in a corner: contours
    # and boxes at the map boundary, then clipped to the source size.
    h, w = 80, 120
    values = np.zeros((h, w), np.float32)
    values[0:4, :] = 0.9
    values[:, 0:4] = 0.9
    values[h - 4:, w - 30:] = 0.8
    transform = (2 * w, 2 * h, w, h)
    (dets,) = gpu.db_postprocess(values, [transform], unclip_ratio=1.5)
    assert len(dets) >= 1
    for d in dets:
        assert np.all(d.polygon >= 0) and np.all(d.polygon[:, 0] <= 2 * w) and np.all(d.polygon[:, 1] <= 2 * h)
    check(dets, values, transform, 2.0, unclip_ratio=1.5)


def test_random_blob_maps_batched(gpu):
    rng = np.random.default_rng(5)
    h, w = 96, 160
    maps = np.stack([blob_map(rng, h, w, 20) for _ in range(3)])
    transforms = [(w * 3, h * 2, w, h), (w, h, w - 7, h - 3), (1000, 700, w - 1, h)]
    out = gpu.db_postprocess(maps, transforms)
    for i in range(3):
        scale = max(transforms[i][0] / transforms[i][2], transforms[i][1] / transforms[i][3])
        check(out[i], maps[i], transforms[i], scale)


def test_isolated_pixels_fill_every_component_slot(gpu):
    # One component per 2x2 block: the most a map can hold.
    h, w = 64, 96
    values = np.zeros((h, w), np.float32)
    values[::2, ::2] = 0.9
    values[::4, ::2] = 0.8  # two score levels
    (dets,) = gpu.db_postprocess(values, [(w, h, w, h)], min_area=1, box_threshold=0.0, max_boxes=10 ** 5)
    assert len(dets) == (h // 2) * (w // 2)
    check(dets, values, (w, h, w, h), min_area=1, box_threshold=0.0, max_boxes=10 ** 5)


def test_max_boxes_keeps_the_highest_scores(gpu):
    rng = np.random.default_rng(9)
    values = np.zeros((120, 200), np.float32)
    for k in range(40):
        y, x = 3 + (k // 8) * 23, 3 + (k % 8) * 24
        values[y:y + 6, x:x + 12] = 0.5 + 0.4 * rng.random()
    (dets,) = gpu.db_postprocess(values, [(200, 120, 200, 120)], max_boxes=7)
    assert len(dets) == 7
    check(dets, values, (200, 120, 200, 120), max_boxes=7)


def test_one_large_component(gpu):
    values = np.full((416, 736), 0.1, np.float32)
    values[8:400, 8:720] = 0.9
    values[100:300:7, 30:700] = 0.3  # striped but connected
    (dets,) = gpu.db_postprocess(values, [(1472, 832, 736, 416)])
    assert len(dets) == 1
    check(dets, values, (1472, 832, 736, 416), scale=2.0)


def test_detector_output_maps(gpu):
    shape = (2, 3, 416, 736)
    x = seeded.seeded_batch(2, 416, 736, 17, detector=True, pattern="blocks")
    det = ppocr_hip.Detector.load(gpu, model_path("det", "tiny"), "tiny", shape)
    transforms = [(1000, 565, 736, 416), (1920, 1080, 736, 414)]
    try:
        maps = det.forward(x).array()[:, 0]
        out = det.detect(x, transforms)
    finally:
        det.close()
    total = 0
    for i in range(2):
        scale = transforms[i][0] / transforms[i][2]
        total += check(out[i], maps[i], transforms[i], scale)
    assert total > 0
    print(f"detector maps: {total} detections")


def test_detect_image_matches_forward_image(gpu):
    img = seeded.seeded_rgb(540, 960, 23, pattern="blocks")
    iw, ih = ppocr_hip.detector_input_plan(960, 540, 736)
    det = ppocr_hip.Detector.load(gpu, model_path("det", "tiny"), "tiny", (1, 3, ih, iw))
    image = gpu.upload_rgb(img)
    corners = quad_corners(0, 0, 960, 540)[None]
    transform = (960, 540, iw, ih)
    try:
        maps = det.forward_image(image, corners).array()[:, 0]
        (dets,) = det.detect_image(image, corners, [transform])
    finally:
        image.close()
        det.close()
    check(dets, maps[0], transform, 960 / iw)


def test_invalid_arguments(gpu):
    values = np.zeros((32, 32), np.float32)
    for kw in [dict(binary_threshold=1.5), dict(min_area=0), dict(max_boxes=0), dict(unclip_ratio=-1.0)]:
        with pytest.raises(ppocr_hip.GpuError) as e:
            gpu.db_postprocess(values, [(32, 32, 32, 32)], **kw)
        assert e.value.kind == "InvalidInput"
    with pytest.raises(ppocr_hip.GpuError):
        gpu.db_postprocess(values, [(32, 0, 32, 32)])
    # extract_detections rejects any non-finite map value, also outside the
    # content area (src/ocr.rs:731-733); the device pass flags it.
    for y, x, v in [(3, 3, np.nan), (31, 31, np.inf), (30, 2, -np.inf), (5, 28, np.nan)]:
        bad = values.copy()
        bad[y, x] = v
        with pytest.raises(ppocr_hip.GpuError) as e:
            gpu.db_postprocess(bad, [(32, 32, 24, 24)])
        assert e.value.kind == "InvalidInput"
    # the flag is cleared between calls: a finite map right after passes
    assert gpu.db_postprocess(values, [(32, 32, 24, 24)]) == [[]]
