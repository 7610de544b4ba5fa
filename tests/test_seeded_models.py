"""The seeded models are informative and well conditioned (CPU oracle only).

Parity is judged within 1e-3 on seeded weights.  That bar only measures
kernel error if the seeded network does not itself amplify fp32 rounding
noise to that size, so each model's output must move by less than a tenth of
the tolerance when the input is perturbed by 1e-7 relative; and its outputs
must not be degenerate (flat map, constant argmax).
"""

import numpy as np
import pytest

import oracle
import seeded
from helpers import model_path

TOL = 1e-3


def perturbed(x, seed=0):
    rng = np.random.default_rng(seed)
    return (x * (1 + rng.uniform(-1e-7, 1e-7, x.shape))).astype(np.float32)


@pytest.mark.parametrize("size", ["tiny", "small", "medium"])
def test_seeded_detector_is_informative_and_conditioned(size):
    m = oracle.Model("det", model_path("det", size), size)
    x = seeded.seeded_batch(1, 128, 224, 7)
    y = m.forward(x)
    assert np.abs(m.forward(perturbed(x)) - y).max() < TOL / 10
    assert y.std() > 0.05
    assert 0.05 < np.mean(y > 0.5) < 0.95


@pytest.mark.parametrize("size", ["tiny", "small", "medium"])
def test_seeded_recognizer_is_informative_and_conditioned(size):
    m = oracle.Model("rec", model_path("rec", size), size)
    x = seeded.seeded_batch(8, 48, 320, 31, detector=False)
    y = m.forward(x)
    assert np.abs(m.forward(perturbed(x)) - y).max() < TOL / 10
    am = y.argmax(-1)
    assert len(np.unique(am)) >= 3
    assert y.max(-1).mean() > 0.2
