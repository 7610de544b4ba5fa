"""Inputs at the edges of what the reference accepts (run on an MI355X).

* Long text lines.  The reference bounds a rectified crop to a 4096-px edge
  (src/ocr.rs:20, :1145-1156), so a recognizer canvas reaches
  48 * 4096 = 196608 px (T = 24576 steps), and its attention has no length
  bound (src/cpu/model.rs:1703-1725).  The small and medium recognizers are
  checked against the oracle at the reference's own 1000x20 -> 2400-px plan
  (src/ocr.rs:1269-1282, T = 300) and on canvases wider than 8192 px
  (T > 1024); the widest canvas runs on the device and is checked through
  size-independent properties (every step a probability distribution; the
  greedy classifier agrees with the probability output).
* Chunked batches.  A plan whose largest buffer would pass the per-buffer
  limit runs its batch in chunks; PPOCR_HIP_MAX_BUFFER_BYTES lowers the limit
  so chunking is exercised at small shapes, against the same model planned
  whole and against the oracle.
"""

import os

import numpy as np
import pytest

import oracle
import ppocr_hip
import seeded
from helpers import argmax_last, ctc_greedy, model_path, quad_corners, synthetic_dictionary

pytestmark = pytest.mark.gpu

REC_TOL = 1e-3
DET_TOL = 1e-3


@pytest.fixture(scope="module")
def gpu():
    g = ppocr_hip.Gpu(0)
    yield g
    g.close()


def check_recognizer(actual, expected):
    assert actual.shape == expected.shape
    err = float(np.max(np.abs(actual - expected)))
    assert err <= REC_TOL, f"max abs diff {err}"
    srt = np.sort(expected, axis=-1)
    clear = (srt[..., -1] - srt[..., -2]) > 1e-4
    assert np.all(argmax_last(actual)[clear] == argmax_last(expected)[clear])
    return err


def test_reference_plan_width_is_2400():
    # recognition_input_plan of the reference's 1000 x 20 literal (src/ocr.rs:1269-1282).
    poly = quad_corners(0, 0, 1000, 20)
    assert ppocr_hip.recognizer_batch_width([poly]) == 2400


@pytest.mark.parametrize("size,batch,width", [
    ("small", 2, 2400),    # the reference's 1000x20 plan, T = 300
    ("medium", 2, 2400),
    ("small", 1, 8320),    # T = 1040 > 1024
    ("medium", 1, 8320),
    ("tiny", 1, 8320),
])
def test_long_line_matches_oracle(gpu, size, batch, width):
    x = seeded.seeded_batch(batch, 48, width, 300 + width, detector=False)
    print(f"long line: {size} [{batch}, 3, 48, {width}]", flush=True)
    rec = ppocr_hip.Recognizer.load(gpu, model_path("rec", size), size, x.shape)
    try:
        out = rec.forward(x).array()
    finally:
        rec.close()
    expected = oracle.Model("rec", model_path("rec", size), size).forward(x)
    err = check_recognizer(out, expected)
    dictionary = synthetic_dictionary(expected.shape[-1])
    for i in range(batch):
        assert ctc_greedy(out[i], dictionary, width, width)[0] == ctc_greedy(expected[i], dictionary, width, width)[0]
    print(f"  max abs {err:.2e}")


@pytest.mark.parametrize("size", ["tiny", "small"])
def test_widest_reference_canvas_runs(gpu, size):
    # 4096 x 1 crop -> canvas 196608 px, T = 24576: too large for the oracle;
    # checked through properties that hold at any size.
    width = 48 * 4096
    x = seeded.seeded_batch(1, 48, width, 77, detector=False)
    print(f"widest canvas: {size} [1, 3, 48, {width}]", flush=True)
    rec = ppocr_hip.Recognizer.load(gpu, model_path("rec", size), size, x.shape)
    greedy = ppocr_hip.Recognizer.load(gpu, model_path("rec", size), size, x.shape, share_weights=rec, greedy=True)
    try:
        probs = rec.forward(x).array()
        steps = greedy.forward(x).array()
    finally:
        greedy.close()
        rec.close()
    assert probs.shape[:2] == (1, width // 8)
    assert np.all(np.isfinite(probs)) and probs.min() >= 0
    assert np.abs(probs.sum(-1) - 1).max() <= 1e-4
    # the fused greedy classifier picks the probability output's argmax
    top2 = np.partition(probs, -2, axis=-1)[..., -2:]
    clear = (top2[..., 1] - top2[..., 0]) > 1e-5
    assert np.all(steps[..., 0].astype(np.int64)[clear] == argmax_last(probs)[clear])
    assert np.abs(steps[..., 1] - probs.max(-1)).max() <= 1e-5


class limited_buffers:
    """Sets PPOCR_HIP_MAX_BUFFER_BYTES while models are loaded (read at load)."""

    def __init__(self, limit):
        self.limit = str(int(limit))

    def __enter__(self):
        os.environ["PPOCR_HIP_MAX_BUFFER_BYTES"] = self.limit

    def __exit__(self, *exc):
        os.environ.pop("PPOCR_HIP_MAX_BUFFER_BYTES", None)


def test_chunked_recognizer_matches_whole_batch(gpu):
    size, batch, width = "small", 5, 320
    x = seeded.seeded_batch(batch, 48, width, 21, detector=False)
    whole = ppocr_hip.Recognizer.load(gpu, model_path("rec", size), size, x.shape)
    # the largest buffer of one line of this plan is the [T, 18710] output
    # (40 * 18710 * 4 B = 3.0 MB): a 7 MB limit plans chunks of two lines
    with limited_buffers(7_000_000):
        part = ppocr_hip.Recognizer.load(gpu, model_path("rec", size), size, x.shape, share_weights=whole)
        part_greedy = ppocr_hip.Recognizer.load(gpu, model_path("rec", size), size, x.shape, share_weights=whole,
                                                greedy=True)
    try:
        assert part.memory_report()["arena_bytes"] < whole.memory_report()["arena_bytes"]
        want = whole.forward(x).array()
        got = part.forward(x).array()
        steps = part_greedy.forward(x).array()
        assert got.shape == want.shape == (batch, 40, 18710)
        assert np.abs(got - want).max() <= 1e-5
        assert np.all(steps[..., 0].astype(np.int64) == argmax_last(want))
        check_recognizer(got, oracle.Model("rec", model_path("rec", size), size).forward(x))
        # device crops, chunked: one image, five quads
        rgb = seeded.seeded_rgb(120, 400, 5)
        img = gpu.upload_rgb(rgb)
        corners = np.stack([quad_corners(10 * i, 5 * i, 10 * i + 300, 5 * i + 40) for i in range(batch)])
        cw = [320, 300, 280, 260, 320]
        a = whole.forward_image(img, corners, cw).array()
        b = part.forward_image(img, corners, cw).array()
        assert np.abs(a - b).max() <= 1e-5
        img.close()
    finally:
        part_greedy.close()
        part.close()
        whole.close()


def test_chunked_detector_matches_whole_batch(gpu):
    size, shape = "tiny", (3, 3, 64, 96)
    x = seeded.seeded_batch(shape[0], shape[2], shape[3], 8, detector=True)
    whole = ppocr_hip.Detector.load(gpu, model_path("det", size), size, shape)
    # one 64 x 96 image's largest buffer is the stem concat (32 x 48 x 32
    # fp32, 196 KB): a 400 KB limit plans chunks of two, the last one partial
    with limited_buffers(400_000):
        part = ppocr_hip.Detector.load(gpu, model_path("det", size), size, shape)
    try:
        assert part.memory_report()["arena_bytes"] < whole.memory_report()["arena_bytes"]
        want = whole.forward(x).array()
        got = part.forward(x).array()
        assert got.shape == want.shape
        assert np.abs(got - want).max() <= 1e-5
        assert np.abs(got - oracle.Model("det", model_path("det", size), size).forward(x)).max() <= DET_TOL
        tr = [(96, 64, 96, 64)] * shape[0]
        d_whole = whole.detect(x, tr)
        d_part = part.detect(x, tr)
        assert [len(d) for d in d_whole] == [len(d) for d in d_part]
        for dw, dp in zip(d_whole, d_part):
            for u, v in zip(dw, dp):
                assert np.abs(u.polygon - v.polygon).max() <= 1e-2 and abs(u.score - v.score) <= 1e-5
    finally:
        part.close()
        whole.close()


def test_one_item_above_the_buffer_limit_is_invalid_input(gpu):
    with limited_buffers(100_000):
        with pytest.raises(ppocr_hip.GpuError) as e:
            ppocr_hip.Recognizer.load(gpu, model_path("rec", "tiny"), "tiny", (2, 3, 48, 320))
    assert e.value.kind == "InvalidInput"
