"""Pins the oracle's bf16 storage emulation, the yardstick of every bf16
tolerance in the GPU parity tests (bf16 storage has no counterpart in the
reference, whose arithmetic is fp32 throughout).

Two things decide what the emulation computes, and each is checked here:
* its rounding function: float32 -> bf16 round-to-nearest-even (NaN kept),
  compared bit for bit with torch's float32 -> bfloat16 conversion on every
  bf16 value (all 2^16 upper halves) with the lower halves that decide the
  rounding (0, 1, just below, at and just above the tie, all ones, and
  random ones), plus subnormals, zeros, infinities and NaN;
* where it rounds: the list of named rounding points the oracle logs in a
  bf16 forward ("A <value>" for an activation rounded to bf16, "W <layer>"
  for weights taken in bf16) must equal, as a multiset, the list the bf16
  plan itself reports (plan_rounding_points, through the test-only probe
  library), for every tier.  The plan's list comes from the storage types of
  the buffers its ops write, so an extra or a missing rounding in the
  emulation, or a fused add the emulation rounds twice, fails here.
"""

import collections
import ctypes

import numpy as np
import pytest

import oracle
import seeded
from helpers import model_path
from test_conv_kernels_gpu import PROBE, bf16_round

SIZE_CODE = {"medium": 0, "small": 1, "tiny": 2}


def _torch_bf16(x):
    torch = pytest.importorskip("torch")
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).to(torch.float32).numpy()


def _all_rounding_cases():
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    lows = [0x0000, 0x0001, 0x7FFE, 0x7FFF, 0x8000, 0x8001, 0xBFFF, 0xFFFF]
    rng = np.random.default_rng(3)
    lows += [int(v) for v in rng.integers(0, 1 << 16, size=8)]
    bits = (hi[:, None] | np.array(lows, dtype=np.uint32)[None, :]).ravel()
    return bits.view(np.float32)


@pytest.mark.parametrize("name,fn", [("oracle", oracle.round_bf16), ("test helper", bf16_round)])
def test_bf16_rounding_matches_torch_bit_for_bit(name, fn):
    x = _all_rounding_cases()
    got = np.asarray(fn(x), dtype=np.float32)
    want = _torch_bf16(x)
    nan = np.isnan(x)
    assert np.array_equal(np.isnan(got), nan), name
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32)), name
    # Spot checks of the cases that tell the rounding rules apart.
    special = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8), 2.0 ** -140, -2.0 ** -149,
                        np.inf, -np.inf, 0.0, -0.0, 3.3895314e38, np.float32(3.4028235e38)], dtype=np.float32)
    np.testing.assert_array_equal(np.asarray(fn(special), dtype=np.float32).view(np.uint32),
                                  _torch_bf16(special).view(np.uint32))
    # Ties go to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7.
    assert float(np.asarray(fn(np.array([1.0 + 2.0 ** -8], np.float32)))[0]) == 1.0


def _plan_rounding(kind, size, shape):
    lib = ctypes.CDLL(str(PROBE))
    fn = lib.ppocr_probe_plan_rounding
    fn.restype = ctypes.c_long
    fn.argtypes = [ctypes.c_char_p] + [ctypes.c_int] * 5 + [ctypes.c_char_p, ctypes.c_size_t]
    path = str(model_path(kind, size)).encode()
    args = (path, 0 if kind == "det" else 1, SIZE_CODE[size], shape[0], shape[2], shape[3])
    n = fn(*args, None, 0)
    assert n > 0, "plan could not be built"
    buf = ctypes.create_string_buffer(n)
    assert fn(*args, buf, n) == n
    return buf.value.decode().splitlines()


def _oracle_rounding(kind, size, shape):
    x = seeded.seeded_batch(shape[0], shape[2], shape[3], 3, detector=(kind == "det"))
    oracle.set_bf16(True)
    try:
        oracle.Model(kind, model_path(kind, size), size).forward(x)
    finally:
        oracle.set_bf16(False)
    return oracle.bf16_log()


CASES = [
    ("det", "tiny", (1, 3, 64, 96)), ("det", "small", (1, 3, 64, 96)), ("det", "medium", (1, 3, 64, 96)),
    ("det", "tiny", (2, 3, 416, 736)), ("det", "medium", (1, 3, 416, 736)),
    ("rec", "tiny", (2, 3, 48, 320)), ("rec", "small", (2, 3, 48, 320)), ("rec", "medium", (2, 3, 48, 320)),
    ("rec", "medium", (3, 3, 48, 96)),
]


@pytest.mark.parametrize("kind,size,shape", CASES, ids=[f"{k}-{s}-{'x'.join(map(str, sh))}" for k, s, sh in CASES])
def test_emulation_rounds_where_the_bf16_plan_rounds(kind, size, shape):
    if not PROBE.exists():
        raise RuntimeError(f"{PROBE} is not built (make -C ppocr-rs_amd)")
    plan = _plan_rounding(kind, size, shape)
    emu = _oracle_rounding(kind, size, shape)
    a, b = collections.Counter(plan), collections.Counter(emu)
    assert a == b, {"plan only": sorted((a - b).elements())[:12], "emulation only": sorted((b - a).elements())[:12]}
    # Every stored tensor of the network is covered: the input, each block,
    # the neck or encoder, and the matrix-core weights of every dense layer.
    assert "A input" in a and any(r.startswith("W ") for r in a)
    assert sum(1 for r in plan if r.startswith("A ")) >= 30
