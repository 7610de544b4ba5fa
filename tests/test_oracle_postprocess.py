"""Pins the oracle's DB postprocess (oracle/postprocess.cpp) before it judges
the device one (CPU only).

Anchors: the reference's own test (src/ocr.rs:1229-1251); 8-connected
components counted independently with scipy.ndimage.label; the closed form
of an axis-aligned rectangle's box (its pixel extent, scaled by unclip about
the centre); mean scores from numpy; the positional sort and the score-based
max_boxes cut.
"""

import numpy as np
import pytest
import scipy.ndimage as ndi

import oracle

EIGHT = np.ones((3, 3), dtype=int)


def test_reference_literal():
    values = np.zeros((416, 736), np.float32)
    values[20:22, 10:14] = 0.9
    polys, scores, _ = oracle.extract_detections(values, (736, 416, 736, 416), min_area=4, unclip_ratio=1.0)
    assert len(scores) == 1
    assert abs(scores[0] - 0.9) < 1e-6
    assert abs(polys[0, 0, 0] - 10.0) < 1e-4


@pytest.mark.parametrize("unclip", [1.0, 1.4, 2.0])
def test_axis_aligned_rectangle_closed_form(unclip):
    values = np.zeros((64, 96), np.float32)
    x0, x1, y0, y1 = 20, 51, 10, 17  # 31 x 7 block
    values[y0:y1, x0:x1] = 0.7
    polys, scores, _ = oracle.extract_detections(values, (96, 64, 96, 64), unclip_ratio=unclip)
    assert len(scores) == 1
    cx, cy = (x0 + x1) / 2, (y0 + y1) / 2
    hw, hh = (x1 - x0) * unclip / 2, (y1 - y0) * unclip / 2
    want = np.array([[cx - hw, cy - hh], [cx + hw, cy - hh], [cx + hw, cy + hh], [cx - hw, cy + hh]])
    assert np.allclose(polys[0], np.clip(want, 0, [96, 64]), atol=1e-3)


def test_components_match_scipy_labelling():
    rng = np.random.default_rng(1)
    for trial in range(10):
        values = (rng.random((40, 60)) < 0.3).astype(np.float32) * 0.9
        _, n = ndi.label(values >= 0.2, structure=EIGHT)
        _, scores, _ = oracle.extract_detections(values, (60, 40, 60, 40), min_area=1, box_threshold=0.0,
                                                 max_boxes=10 ** 6)
        assert len(scores) == n


def test_filters_and_scores_match_numpy():
    rng = np.random.default_rng(2)
    values = rng.random((50, 70)).astype(np.float32) * 0.3
    for _ in range(15):
        y, x = rng.integers(0, 45), rng.integers(0, 60)
        values[y:y + rng.integers(1, 6), x:x + rng.integers(1, 10)] = rng.uniform(0.2, 1.0)
    lab, n = ndi.label(values >= 0.2, structure=EIGHT)
    want = []
    for k in range(1, n + 1):
        sel = lab == k
        score = np.float32(values[sel].astype(np.float64).mean())
        if sel.sum() >= 3 and score >= 0.4:
            want.append(score)
    _, scores, _ = oracle.extract_detections(values, (70, 50, 70, 50))
    assert sorted(np.round(scores, 6)) == sorted(np.round(want, 6))


def test_content_rectangle_limits_the_search_and_maps_to_source():
    values = np.zeros((32, 64), np.float32)
    values[4:8, 4:12] = 0.8   # inside the 40 x 20 content
    values[4:8, 50:60] = 0.8  # outside it: ignored
    polys, scores, _ = oracle.extract_detections(values, (400, 100, 40, 20), unclip_ratio=1.0)
    assert len(scores) == 1
    # content x 4..12 -> source x 40..120; content y 4..8 -> source y 20..40.
    assert np.allclose(polys[0], [[40, 20], [120, 20], [120, 40], [40, 40]], atol=1e-3)


def test_positional_order_and_max_boxes():
    values = np.zeros((60, 60), np.float32)
    blocks = [(40, 5, 0.5), (5, 40, 0.9), (5, 5, 0.6), (40, 40, 0.95), (22, 22, 0.45)]
    for y, x, s in blocks:
        values[y:y + 4, x:x + 4] = s
    polys, scores, _ = oracle.extract_detections(values, (60, 60, 60, 60))
    centers = polys.mean(1)
    order = np.lexsort((centers[:, 0], centers[:, 1]))
    assert np.array_equal(order, np.arange(len(scores)))
    assert np.allclose(sorted(scores), sorted(s for _, _, s in blocks), atol=1e-6)
    _, top, _ = oracle.extract_detections(values, (60, 60, 60, 60), max_boxes=2)
    assert sorted(top) == pytest.approx(sorted([0.9, 0.95]), abs=1e-6)


def test_rotated_bar_axis():
    # A diagonal bar symmetric under x <-> y (pixels with |x - y| <= 1): its
    # covariance has cov_xx == cov_yy, so the fitted box follows 45 degrees.
    values = np.zeros((80, 80), np.float32)
    yy, xx = np.mgrid[0:80, 0:80]
    values[(np.abs(xx - yy) <= 1) & (xx >= 10) & (xx < 60) & (yy >= 10) & (yy < 60)] = 0.9
    polys, _, aniso = oracle.extract_detections(values, (80, 80, 80, 80), unclip_ratio=1.0)
    edge = polys[0, 1] - polys[0, 0]
    assert abs(abs(edge[0]) - abs(edge[1])) < 1e-3 * np.abs(edge).max()
    assert aniso[0] > 0.9


def test_invalid_options_are_rejected():
    values = np.zeros((8, 8), np.float32)
    for kw in [dict(binary_threshold=1.5), dict(min_area=0), dict(max_boxes=0), dict(unclip_ratio=0.0)]:
        with pytest.raises(ValueError):
            oracle.extract_detections(values, (8, 8, 8, 8), **kw)
    bad = values.copy()
    bad[1, 1] = np.inf
    with pytest.raises(ValueError):
        oracle.extract_detections(bad, (8, 8, 8, 8))
