"""Input plans and the greedy-CTC collapse of the C ABI (host code, no GPU).

Pinned by the reference's own literal tests (src/preprocess.rs:150-179,
src/ocr.rs:1254-1301) and by what the arithmetic fixes: aligned sides are the
nearest multiple of 32, content widths are ceil(48 w / h) of the bounded crop,
the batch canvas is the largest content width (at least 320) rounded up to a
multiple of 4, and the decode emits a class on each change away from blank
with score exp(mean ln p).
"""

import math

import numpy as np
import pytest

import oracle
import ppocr_hip
from helpers import quad_corners


def rect(w, h, x=0.0, y=0.0):
    return quad_corners(x, y, x + w, y + h)


# ------------------------------------------------------------ detector plan

def test_detector_plan_matches_reference_literal():
    # src/preprocess.rs:150-158: 1920x1080 with the default 736 limit.
    assert ppocr_hip.detector_input_plan(1920, 1080, 736) == (736, 416)


@pytest.mark.parametrize("w,h,limit", [(640, 480, 736), (100, 3000, 736), (4000, 37, 960), (31, 31, 736),
                                       (1000, 1000, 2000), (737, 736, 736)])
def test_detector_plan_with_limit_is_the_nearest_multiple_of_32(w, h, limit):
    ratio = min(limit / max(w, h), 1.0)
    got = ppocr_hip.detector_input_plan(w, h, limit)
    for side, src in zip(got, (w, h)):
        assert side % 32 == 0 and side >= 32
        if src * ratio >= 16:
            assert abs(side - src * ratio) <= 16 + 1e-9
        else:
            assert side == 32


def test_detector_plan_default_ratio():
    # default_detector_ratio: short side raised to 736, long side capped at 4000.
    assert ppocr_hip.detector_input_plan(368, 184, None) == (1472, 736)
    assert ppocr_hip.detector_input_plan(1920, 1080, None) == (1920, 1088)
    # 100 x 10000: 7.36x would give 73600 > 4000, so the ratio is 0.4.
    assert ppocr_hip.detector_input_plan(100, 10000, None) == (32, 4000)


def test_detector_plan_rejects_bad_arguments():
    with pytest.raises(ppocr_hip.GpuError) as e:
        ppocr_hip.detector_input_plan(100, 100, 0)
    assert e.value.kind == "InvalidInput"
    with pytest.raises(ppocr_hip.GpuError):
        ppocr_hip.detector_input_plan(0, 100, 736)


# ------------------------------------------------------------ recognizer plan

def test_recognizer_plan_matches_reference_literals():
    # src/preprocess.rs:161-179: an 80x20 crop has content width 192 of 320.
    assert ppocr_hip.recognition_input_plan(rect(80, 20), 320) == 192
    # src/ocr.rs:1284-1301: the widest crop sets the canvas.
    assert ppocr_hip.recognizer_batch_width([rect(80, 20), rect(300, 20)]) == 720
    # src/ocr.rs:1269-1282: a 1000x20 crop keeps its whole width.
    wide = rect(1000, 20)
    width = ppocr_hip.recognizer_batch_width([wide])
    assert width == 2400
    assert ppocr_hip.recognition_input_plan(wide, width) == 2400


@pytest.mark.parametrize("w,h", [(1, 1), (7, 3), (33, 48), (500, 17), (48, 48), (95, 32), (10, 200)])
def test_content_width_is_the_ceiling_of_48_w_over_h(w, h):
    c = ppocr_hip.recognition_input_plan(rect(w, h, 5.0, 9.0), 1 << 20)
    assert c * h >= 48 * w and (c - 1) * h < 48 * w


def test_batch_width_is_the_rounded_maximum():
    quads = [rect(81, 20), rect(70, 20)]
    # 48 * 81 / 20 = 194.4 -> 195 < 320, so the canvas stays 320.
    assert ppocr_hip.recognizer_batch_width(quads) == 320
    # 48 * 401 / 20 = 962.4 -> 963 -> rounded up to 964.
    assert ppocr_hip.recognizer_batch_width(quads + [rect(401, 20)]) == 964
    assert ppocr_hip.recognizer_batch_width(np.zeros((0, 4, 2), np.float32)) == 320


def test_rotated_crop_uses_the_longer_opposite_edges():
    # A parallelogram: top edge 100, bottom edge 120 long; left and right 30.
    q = np.array([[0, 0], [100, 0], [120, 30], [0, 30]], np.float32)
    right = math.sqrt(20 * 20 + 30 * 30)
    c = ppocr_hip.recognition_input_plan(q, 1 << 20)
    assert c == math.ceil(48 * 120 / round(right))


def test_crop_is_bounded_to_the_rectified_limits():
    # 5000 x 10: the 4096 edge limit scales it by 0.8192 -> 4096 x 8.
    assert ppocr_hip.recognition_input_plan(rect(5000, 10), 1 << 20) == 48 * 4096 // 8
    # 4000 x 4000: the 8e6 pixel limit scales by sqrt(0.5) -> 2828 x 2828.
    assert ppocr_hip.recognition_input_plan(rect(4000, 4000), 1 << 20) == 48


def test_recognizer_plan_rejects_bad_crops():
    with pytest.raises(ppocr_hip.GpuError) as e:
        ppocr_hip.recognition_input_plan(rect(0, 20), 320)
    assert e.value.kind == "InvalidInput"
    with pytest.raises(ppocr_hip.GpuError):
        ppocr_hip.recognition_input_plan(rect(400, 20), 320)  # 960 > 320
    bad = rect(10, 10)
    bad[1, 0] = np.nan
    with pytest.raises(ppocr_hip.GpuError):
        ppocr_hip.recognizer_batch_width([bad])


# ------------------------------------------------------------ greedy CTC

def steps_of(rows):
    """(class, probability) pairs of probability rows, the form a greedy
    recognizer writes."""
    rows = np.asarray(rows, np.float32)
    cls = rows.shape[1] - 1 - np.argmax(rows[:, ::-1], axis=1)
    return np.stack([cls.astype(np.float32), rows[np.arange(len(rows)), cls]], axis=1)


def test_ctc_matches_reference_literal():
    # src/ocr.rs:1254-1266: five steps of "A", only ceil(40 * 5 / 100) = 2 valid.
    rows = np.array([[0.1, 0.9]] * 5, np.float32)
    d = ppocr_hip.ctc_greedy_decode(steps_of(rows), ["A"], 2, 40, 100)
    assert d.text == "A"
    assert abs(d.score - 0.9) < 1e-6
    assert oracle.ctc_greedy_decode(rows, 1, 40, 100) == ([1], pytest.approx(0.9, abs=1e-6))


def test_ctc_collapses_repeats_and_blanks():
    # classes: 0 blank, 1 'a', 2 'b'; path a a _ a b b _ -> "aab".
    path = [1, 1, 0, 1, 2, 2, 0]
    probs = [0.9, 0.8, 0.99, 0.7, 0.6, 0.95, 0.9]
    steps = np.array(list(zip(path, probs)), np.float32)
    d = ppocr_hip.ctc_greedy_decode(steps, ["a", "b"], 3, 320, 320)
    assert d.text == "aab"
    want = math.exp((math.log(np.float32(0.9)) + math.log(np.float32(0.7)) + math.log(np.float32(0.6))) / 3)
    assert abs(d.score - want) < 1e-6


def test_ctc_implicit_space_and_empty_output():
    steps = np.array([[2, 0.5], [1, 0.5], [2, 0.5]], np.float32)
    assert ppocr_hip.ctc_greedy_decode(steps, ["x"], 3, 3, 3).text == " x "
    blank = np.array([[0, 0.9]] * 4, np.float32)
    d = ppocr_hip.ctc_greedy_decode(blank, ["x"], 2, 4, 4)
    assert d.text == "" and d.score == 0.0


def test_ctc_probability_floor():
    steps = np.array([[1, 0.0]], np.float32)
    assert abs(ppocr_hip.ctc_greedy_decode(steps, ["a"], 2, 1, 1).score - 1e-8) < 1e-12


def test_ctc_rejects_inconsistent_arguments():
    steps = np.array([[1, 0.9]], np.float32)
    for classes, dict_len, cw, iw in [(5, 1, 1, 1), (2, 1, 0, 1), (2, 1, 3, 2)]:
        with pytest.raises(ppocr_hip.GpuError) as e:
            ppocr_hip.ctc_greedy_decode(steps, ["a"] * dict_len, classes, cw, iw)
        assert e.value.kind == "InvalidInput"
    with pytest.raises(ppocr_hip.GpuError):
        ppocr_hip.ctc_greedy_decode(np.array([[7, 0.9]], np.float32), ["a"], 2, 1, 1)


def test_ctc_decode_of_steps_equals_oracle_on_rows():
    rng = np.random.default_rng(3)
    dictionary = [chr(ord("a") + i) for i in range(9)]
    for trial in range(40):
        t, v = 40, 10 + (trial % 2)  # V = dict + 1, or dict + 2 (implicit space)
        logits = rng.normal(0, 2, (t, v)).astype(np.float32)
        logits[rng.random(t) < 0.3, 0] += 4  # plenty of blanks
        e = np.exp(logits - logits.max(1, keepdims=True))
        rows = (e / e.sum(1, keepdims=True)).astype(np.float32)
        if trial % 5 == 0:  # exact ties resolve to the last index
            rows[3, 2] = rows[3, 5] = rows[3].max() + 0.01
            rows[3] /= rows[3].sum()  # still a distribution; equal values stay equal
        cw, iw = int(rng.integers(1, 321)), 320
        tokens, score = oracle.ctc_greedy_decode(rows, len(dictionary), cw, iw)
        d = ppocr_hip.ctc_greedy_decode(steps_of(rows), dictionary, v, cw, iw)
        text = "".join(" " if v == len(dictionary) + 2 and c == v - 1 else dictionary[c - 1] for c in tokens)
        assert d.text == text
        assert abs(d.score - score) <= 1e-6 * max(1.0, score)


def test_oracle_ctc_uses_softmax_for_non_distributions():
    # Logit rows (not a distribution): the probability is the row's softmax.
    rows = np.array([[0.0, 2.0, 1.0]], np.float32)
    tokens, score = oracle.ctc_greedy_decode(rows, 2, 1, 1)
    e = np.exp([0.0, 2.0, 1.0])
    assert tokens == [1] and abs(score - e[1] / e.sum()) < 1e-6
