"""Shared helpers of the test suite: seeded model files, comparison rules and
the CPU-side reference decoders used for the exact-output checks."""

from __future__ import annotations

import pathlib
import tempfile

import numpy as np

import oracle
import seeded

_CACHE = pathlib.Path(tempfile.gettempdir()) / "ppocr_hip_test_models"


def model_path(kind, size, seed=None):
    """Seeded safetensors file for (kind, size), generated once per machine."""
    seed = (1 if kind == "det" else 2) if seed is None else seed
    _CACHE.mkdir(parents=True, exist_ok=True)
    gain, head_gain = seeded.DEFAULT_GAINS[(kind, size)]
    path = _CACHE / f"{kind}_{size}_s{seed}_g{gain}_{head_gain}.safetensors"
    if not path.exists():
        tmp = path.with_suffix(".tmp")
        seeded.write_weights(tmp, kind, size, seed=seed)
        tmp.replace(path)
    return path


def band_mismatches(actual, expected, threshold, eps=1e-5):
    """Binarisation mismatches at `threshold` outside the ambiguity band.

    Values within `eps` of the threshold may legitimately round to either
    side; everything else must agree exactly.  Returns (mismatches, band).
    """
    a = actual >= threshold
    e = expected >= threshold
    band = np.abs(expected - threshold) <= eps
    return int(np.count_nonzero((a != e) & ~band)), int(np.count_nonzero(band))


def argmax_last(rows):
    """Argmax with ties resolved to the last index, as Rust's
    ``max_by(total_cmp)`` (src/bin/benchmark.rs:287-293, src/ocr.rs:1171-1177)."""
    rows = np.asarray(rows)
    flipped = rows[..., ::-1]
    return rows.shape[-1] - 1 - np.argmax(flipped, axis=-1)


def ctc_greedy(probs, dictionary, content_width, input_width):
    """The oracle's ``decode_ctc_greedy_for_input`` (src/ocr.rs:800-853) for one
    [T, V] item, with the tokens mapped through `dictionary`."""
    classes = probs.shape[1]
    tokens, score = oracle.ctc_greedy_decode(probs, len(dictionary), content_width, input_width)
    space = classes == len(dictionary) + 2
    return "".join(" " if space and c == classes - 1 else dictionary[c - 1] for c in tokens), score


def synthetic_dictionary(classes):
    """Dictionary of `classes - 1` distinct tokens (blank is class 0)."""
    return [f"<{i}>" for i in range(1, classes)]


def quad_corners(x0, y0, x1, y1):
    return np.array([[x0, y0], [x1, y0], [x1, y1], [x0, y1]], dtype=np.float32)


def edit_distance(a, b):
    """Levenshtein distance between two token sequences."""
    prev = list(range(len(b) + 1))
    for i, x in enumerate(a, 1):
        cur = [i]
        for j, y in enumerate(b, 1):
            cur.append(min(prev[j] + 1, cur[j - 1] + 1, prev[j - 1] + (x != y)))
        prev = cur
    return prev[-1]
