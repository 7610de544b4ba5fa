"""Kernel-level checks of the depthwise convolutions on the GPU.

The bf16 matrix-core depthwise (5x5, 7x7, 9x9 as Toeplitz products of tap
rows) and the VALU kernels run through the test harness
libppocr_hip_probe.so on maps whose sides are not multiples of the tiles,
and are compared with a float64 depthwise of the same operands (zero
padding k / 2, bias, activation, then the residual: the reference depthwise
semantics, src/cpu/ops.rs and the scalar references of
src/cpu/kernels/mod.rs:2880-2997).  Each case first asserts which kernel
instance it runs.
"""
import ctypes

import numpy as np
import pytest

from test_conv_kernels_gpu import ACT_HSWISH, ACT_NONE, ACT_RELU, PROBE, _ptr, act, bf16_round


def _lib():
    if not PROBE.exists():
        raise RuntimeError(f"{PROBE} is not built (make -C ppocr-rs_amd)")
    lib = ctypes.CDLL(str(PROBE))
    f = ctypes.POINTER(ctypes.c_float)
    i = ctypes.c_int
    lib.ppocr_probe_depthwise.argtypes = [f, i, i, i, i, f, f, i, i, f, i, i, f]
    lib.ppocr_probe_depthwise.restype = i
    lib.ppocr_probe_depthwise_kernel.argtypes = [i, i, i, i, i]
    lib.ppocr_probe_depthwise_kernel.restype = ctypes.c_char_p
    return lib


def depthwise_ref(x, w, b, kind, res):
    """float64 NHWC depthwise, stride 1, pads k // 2: x [n][h][w][c], w [c][k][k]."""
    n, h, wd, c = x.shape
    k = w.shape[-1]
    p = k // 2
    xp = np.zeros((n, h + 2 * p, wd + 2 * p, c))
    xp[:, p:p + h, p:p + wd] = x
    y = np.zeros((n, h, wd, c))
    for ky in range(k):
        for kx in range(k):
            y += xp[:, ky:ky + h, kx:kx + wd, :] * w[:, ky, kx].astype(np.float64)
    if b is not None:
        y += b
    y = act(y, kind)
    if res is not None:
        y += res
    return y


# (n, h, w, c, k, act, bias, residual): tails in both directions, one and
# several 8-channel groups, maps taller than one 32-row tile.
MFMA_CASES = [
    (1, 16, 16, 8, 9, ACT_NONE, False, False),
    (2, 37, 45, 24, 9, ACT_NONE, False, False),
    (1, 70, 33, 72, 9, ACT_RELU, True, False),
    (1, 29, 71, 8, 7, ACT_HSWISH, True, True),
    (2, 18, 40, 16, 5, ACT_NONE, True, True),
    (1, 52, 92, 16, 5, ACT_RELU, False, False),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", MFMA_CASES, ids=lambda c: "x".join(map(str, c[:5])))
def test_bf16_matrix_core_depthwise_matches_float64(case):
    n, h, wd, c, k, kind, has_bias, has_res = case
    lib = _lib()
    kernel = lib.ppocr_probe_depthwise_kernel(h, c, k, 1, 1).decode()
    assert kernel == f"depthwise_mfma<{k}x{k}>", kernel
    rng = np.random.default_rng(1000 + 7 * h + wd + k)
    x = rng.uniform(-1, 1, (n, h, wd, c)).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (c, k, k)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, c).astype(np.float32) if has_bias else None
    res = rng.uniform(-1, 1, (n, h, wd, c)).astype(np.float32) if has_res else None
    out = np.zeros((n, h, wd, c), np.float32)
    assert lib.ppocr_probe_depthwise(_ptr(x), n, h, wd, c, _ptr(w), _ptr(b), k, kind, _ptr(res), 1, 1, _ptr(out)) == 0
    # The kernel multiplies bf16 activations by bf16 taps exactly and sums in
    # fp32, then stores bf16: against the float64 result of the same rounded
    # operands the error is the output rounding (2^-9 relative) plus the fp32
    # sum of k * k terms.
    ref = depthwise_ref(bf16_round(x), bf16_round(w), b, kind, None if res is None else bf16_round(res))
    err = np.abs(out - ref)
    tol = 2.0 ** -8 * np.abs(ref) + 1e-4
    assert np.all(err <= tol), (float(err.max()), np.unravel_index(np.argmax(err - tol), err.shape))


@pytest.mark.gpu
@pytest.mark.parametrize("k", [5, 7, 9])
def test_matrix_core_and_valu_depthwise_agree(k):
    """The same bf16 layer without the packed taps runs the VALU kernel (fp32
    taps); the two differ only by the taps' bf16 rounding and summation order."""
    lib = _lib()
    n, h, wd, c = 2, 41, 57, 24
    assert lib.ppocr_probe_depthwise_kernel(h, c, k, 1, 0).decode() != f"depthwise_mfma<{k}x{k}>"
    rng = np.random.default_rng(k)
    x = rng.uniform(-1, 1, (n, h, wd, c)).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (c, k, k)).astype(np.float32)
    outs = []
    for table in (1, 0):
        out = np.zeros((n, h, wd, c), np.float32)
        assert lib.ppocr_probe_depthwise(_ptr(x), n, h, wd, c, _ptr(w), None, k, ACT_NONE, None, 1, table,
                                         _ptr(out)) == 0
        outs.append(out)
    ref = depthwise_ref(bf16_round(x), w, None, ACT_NONE, None)
    scale = np.sqrt(k * k) * 0.5 * 2.0 ** -8  # bf16 tap rounding, summed over k * k random-sign terms
    for out in outs:
        assert np.abs(out - ref).max() <= 2.0 ** -8 * np.abs(ref).max() + 4 * scale


@pytest.mark.gpu
def test_matrix_core_depthwise_needs_whole_channel_groups():
    """12 channels (not a multiple of 8) and maps under 16 rows stay on the
    VALU kernels; their outputs still match float64."""
    lib = _lib()
    assert lib.ppocr_probe_depthwise_kernel(30, 12, 9, 1, 1).decode() == "depthwise_wave<9x9>"
    assert lib.ppocr_probe_depthwise_kernel(12, 16, 5, 1, 1).decode() == "depthwise_wave<5x5>"
    for n, h, wd, c, k in ((1, 30, 41, 12, 9), (2, 12, 40, 16, 5)):
        rng = np.random.default_rng(h + c)
        x = rng.uniform(-1, 1, (n, h, wd, c)).astype(np.float32)
        w = rng.uniform(-0.5, 0.5, (c, k, k)).astype(np.float32)
        out = np.zeros((n, h, wd, c), np.float32)
        assert lib.ppocr_probe_depthwise(_ptr(x), n, h, wd, c, _ptr(w), None, k, ACT_NONE, None, 1, 1, _ptr(out)) == 0
        ref = depthwise_ref(bf16_round(x), w, None, ACT_NONE, None)
        assert np.all(np.abs(out - ref) <= 2.0 ** -8 * np.abs(ref) + 1e-4)


@pytest.mark.gpu
def test_fp32_depthwise_probe_matches_float64():
    """The probe's fp32 path (VALU kernels: tiled 3x3 and 7x7, wave 5x5 and
    9x9) against float64: pins the probe."""
    lib = _lib()
    for k in (3, 5, 7, 9):
        n, h, wd, c = 1, 23, 35, 8
        rng = np.random.default_rng(50 + k)
        x = rng.uniform(-1, 1, (n, h, wd, c)).astype(np.float32)
        w = rng.uniform(-0.5, 0.5, (c, k, k)).astype(np.float32)
        b = rng.uniform(-0.5, 0.5, c).astype(np.float32)
        out = np.zeros((n, h, wd, c), np.float32)
        assert lib.ppocr_probe_depthwise(_ptr(x), n, h, wd, c, _ptr(w), _ptr(b), k, ACT_RELU, None, 0, 0,
                                         _ptr(out)) == 0
        ref = depthwise_ref(x, w, b, ACT_RELU, None)
        assert np.abs(out - ref).max() <= 1e-5


# (k, n, h, w, c, with upper level): the RepLK FPN's input-conv layers with
# the gate-residual formed in the tile loads (5x5 wave, 7x7 tiled, 9x9 wave).
GR_CASES = [(5, 1, 26, 46, 64, True), (5, 2, 13, 23, 32, False), (7, 1, 20, 34, 96, True), (9, 1, 18, 22, 16, True)]


@pytest.mark.gpu
@pytest.mark.parametrize("case", GR_CASES, ids=[f"k{c[0]}-{c[2]}x{c[3]}x{c[4]}{'-up' if c[5] else ''}" for c in GR_CASES])
def test_gate_residual_prologue_matches_float64(case):
    k, n, h, wd, c, with_up = case
    lib = _lib()
    f = ctypes.POINTER(ctypes.c_float)
    i = ctypes.c_int
    lib.ppocr_probe_depthwise_gate_residual.argtypes = [f, i, i, i, i, f, f, f, f, i, f, f]
    lib.ppocr_probe_depthwise_gate_residual.restype = i
    rng = np.random.default_rng(1000 * k + h)
    hx = rng.standard_normal((n, h, wd, c)).astype(np.float32)
    gate = rng.uniform(0, 1, (n, c)).astype(np.float32)
    up = rng.standard_normal((n, h // 2, wd // 2, c)).astype(np.float32) if with_up else None
    w = (rng.standard_normal((c, k, k)) / k).astype(np.float32)
    b = rng.standard_normal(c).astype(np.float32) * 0.1
    out = np.empty((n, h, wd, c), np.float32)
    xout = np.empty((n, h, wd, c), np.float32)
    assert lib.ppocr_probe_depthwise_gate_residual(_ptr(hx), n, h, wd, c, _ptr(gate), _ptr(up), _ptr(w), _ptr(b), k,
                                                   _ptr(out), _ptr(xout)) == 0
    # x = h + h*g with both roundings in fp32 (the reference's two-step
    # residual multiply), then + up2(upper) in fp32: bit-exact.
    x = (hx * gate[:, None, None, :]).astype(np.float32) + hx
    if with_up:
        x = x + np.repeat(np.repeat(up, 2, axis=1), 2, axis=2)
    bad = np.argwhere(xout != x)
    assert bad.size == 0, f"{len(bad)} of {x.size} differ, first {bad[:3].tolist()}: {xout[tuple(bad[0])]} vs {x[tuple(bad[0])]}"
    # float64 depthwise of x.
    pd = k // 2
    xp = np.pad(x.astype(np.float64), ((0, 0), (pd, pd), (pd, pd), (0, 0)))
    want = np.zeros((n, h, wd, c))
    for ky in range(k):
        for kx in range(k):
            want += xp[:, ky:ky + h, kx:kx + wd, :] * w[:, ky, kx]
    want += b
    err = np.abs(out - want)
    assert np.all(err <= 1e-5 + 1e-5 * np.abs(want)), f"max err {err.max()}"


@pytest.mark.gpu
def test_gelu_epilogue_at_infinities_and_large_values():
    """The device GELU (A-S erf form, shared by every kernel's epilogue)
    follows v/2 (1 + erf(v / sqrt 2)) where it overflows: +inf stays +inf,
    -inf gives NaN (-inf times 0), NaN stays NaN, large finite values give v
    (positive) or 0 (negative).  Run as a 3x3 depthwise with only its centre
    tap set, over 1x1 maps, so each value meets only zero padding."""
    ACT_GELU = 2
    lib = _lib()
    vals = np.array([np.inf, -np.inf, np.nan, 3.0e38, -3.0e38, 1.0e30, -1.0e30, 1.0e6, -1.0e6, 40.0, -40.0, 0.0,
                     1.0, -1.0, 0.5, -0.5], np.float32)
    n, c = 4, 16
    x = np.resize(vals, n * c).reshape(n, 1, 1, c).astype(np.float32)
    w = np.zeros((c, 3, 3), np.float32)
    w[:, 1, 1] = 1.0
    out = np.empty_like(x)
    assert lib.ppocr_probe_depthwise(_ptr(x), n, 1, 1, c, _ptr(w), None, 3, ACT_GELU, None, 0, 0, _ptr(out)) == 0
    v = x.ravel().astype(np.float64)
    got = out.ravel()
    import math

    exact = np.array([0.5 * t * (1.0 + math.erf(t / math.sqrt(2.0))) if np.isfinite(t) else np.nan for t in v])
    for t, g, e in zip(v, got, exact):
        if np.isnan(t) or t == -np.inf:
            assert np.isnan(g), (t, g)
        elif t == np.inf:
            assert g == np.inf, (t, g)
        else:
            assert np.isfinite(g), (t, g)
            assert abs(g - e) <= 1e-6 * abs(e) + 1e-6, (t, g, e)


# (n, h, w, c, act, bias, residual): the bf16 3x3 tiled kernel with 8
# channels per lane, on maps whose height is a multiple of 4 but not of 8
# or is 3 (4-row tiles, 16 pixels wide), of 6 rows (2-row tiles, 32 wide)
# and others (8-row tiles, 8 pixels wide), with row, column and
# channel-block tails.
TILED8_CASES = [
    (2, 6, 80, 64, ACT_NONE, True, False),
    (4, 3, 80, 96, ACT_NONE, True, True),
    (2, 4, 19, 24, ACT_RELU, True, False),
    (1, 12, 37, 72, ACT_HSWISH, True, True),
    (3, 7, 21, 8, ACT_RELU, False, True),
    (1, 29, 45, 136, ACT_NONE, True, False),
    (2, 17, 9, 16, ACT_HSWISH, False, False),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", TILED8_CASES, ids=lambda c: "x".join(map(str, c[:4])))
def test_bf16_tiled8_depthwise_matches_float64(case):
    """bf16 activations (rounded on store), fp32 taps and sums: against the
    float64 depthwise of the bf16-rounded input the error is the output
    rounding (2^-9 relative) plus the fp32 sums of nine products."""
    n, h, wd, c, kind, has_bias, has_res = case
    lib = _lib()
    kernel = lib.ppocr_probe_depthwise_kernel(h, c, 3, 1, 0).decode()
    assert kernel == "depthwise_tiled8<3x3>", kernel
    rng = np.random.default_rng(77 + 3 * h + wd + c)
    x = rng.uniform(-1, 1, (n, h, wd, c)).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (c, 3, 3)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, c).astype(np.float32) if has_bias else None
    res = rng.uniform(-1, 1, (n, h, wd, c)).astype(np.float32) if has_res else None
    out = np.empty_like(x)
    assert lib.ppocr_probe_depthwise(_ptr(x), n, h, wd, c, _ptr(w), _ptr(b), 3, kind, _ptr(res), 1, 0, _ptr(out)) == 0
    ref = depthwise_ref(bf16_round(x), w, b, kind, None if res is None else bf16_round(res))
    err = np.abs(out - ref)
    tol = 2.0 ** -8 * np.abs(ref) + 1e-5
    assert np.all(err <= tol), (float(err.max()), np.unravel_index(np.argmax(err - tol), err.shape))
    # Every output is finite and written (no stale pixels past the tiles).
    assert np.all(np.isfinite(out))


# (n, h, w, c, dt, rows per image): the SE channel sums the tiled 3x3
# kernels leave with their outputs, one row per tile of an image.  bf16 maps
# of 3 or 4 rows, or whose height is a multiple of 4 but not of 8, take
# 4-row tiles 16 pixels wide, 6-row ones 2-row tiles 32 pixels wide, the
# others 8-row tiles 8 pixels wide (fp32 always).
DW_SE_CASES = [
    (3, 12, 80, 128, 1, 5 * 3),
    (2, 6, 37, 64, 1, 2 * 3),
    (1, 6, 80, 512, 1, 3 * 3),
    (2, 3, 80, 768, 1, 5 * 1),
    (1, 4, 21, 64, 1, 2 * 1),
    (1, 52, 92, 256, 1, 6 * 13),
    (2, 29, 45, 72, 1, 6 * 4),
    (2, 12, 40, 32, 0, 5 * 2),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", DW_SE_CASES, ids=lambda c: "x".join(map(str, c[:4])) + ("-bf16" if c[4] else "-f32"))
def test_tiled_depthwise_se_sums_match_stored_outputs(case):
    """Summed over an image's rows, the partial sums equal the channel sums
    of the stored (rounded) outputs up to fp32 summation order, and there
    is one row per tile of the image."""
    n, h, wd, c, dt, want_rows = case
    lib = _lib()
    f = ctypes.POINTER(ctypes.c_float)
    i = ctypes.c_int
    lib.ppocr_probe_depthwise_se.argtypes = [f, i, i, i, i, f, f, i, i, f, ctypes.POINTER(i), f]
    lib.ppocr_probe_depthwise_se.restype = i
    rng = np.random.default_rng(5 + h + wd + c + dt)
    x = rng.uniform(-1, 1, (n, h, wd, c)).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (c, 3, 3)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, c).astype(np.float32)
    out = np.empty_like(x)
    rows = ctypes.c_int(0)
    part = np.full((n * (h // 4 + 1) * (wd // 8 + 1), c), np.nan, np.float32)
    assert lib.ppocr_probe_depthwise_se(_ptr(x), n, h, wd, c, _ptr(w), _ptr(b), ACT_NONE, dt, _ptr(out),
                                        ctypes.byref(rows), _ptr(part)) == 0
    assert rows.value == want_rows
    sums = part[:n * rows.value].reshape(n, rows.value, c).astype(np.float64).sum(axis=1)
    want = out.astype(np.float64).sum(axis=(1, 2))
    scale = np.abs(out).astype(np.float64).sum(axis=(1, 2))
    assert np.all(np.abs(sums - want) <= 1e-5 * scale + 1e-6), float(np.max(np.abs(sums - want) / (scale + 1)))
    ref = depthwise_ref(bf16_round(x) if dt else x, w, b, ACT_NONE, None)
    tol = (2.0 ** -8 if dt else 1e-5) * np.abs(ref) + 1e-5
    assert np.all(np.abs(out - ref) <= tol)


# (n, h, w, c, sh, sw, dt, kernel): 3x3 stage-entry depthwise layers (pads
# 1) with vertical stride 2 on the tiled kernels (bf16 on the 8-channel
# form, fp32 on the 4-channel one): stride (2, 1), the recognizer's, with
# the output height's tile rows; stride (2, 2), the detector's, with 4-row
# tiles; row, column and channel-block tails.
DW_STRIDED_CASES = [
    (4, 12, 80, 256, 2, 1, 1, "depthwise_tiled8<3x3,s2>"),
    (4, 6, 37, 64, 2, 1, 1, "depthwise_tiled8<3x3,s2>"),
    (2, 13, 23, 96, 2, 1, 1, "depthwise_tiled8<3x3,s2>"),
    (2, 52, 92, 128, 2, 2, 1, "depthwise_tiled8<3x3,s2>"),
    (1, 27, 45, 24, 2, 2, 1, "depthwise_tiled8<3x3,s2>"),
    (2, 12, 30, 32, 2, 2, 0, "depthwise_tiled<3x3,s2>"),
    (3, 13, 41, 36, 2, 2, 0, "depthwise_tiled<3x3,s2>"),
    (4, 6, 50, 96, 2, 1, 0, "depthwise_tiled<3x3,s2>"),
    (4, 12, 21, 48, 2, 1, 0, "depthwise_tiled<3x3,s2>"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", DW_STRIDED_CASES,
                         ids=lambda c: "x".join(map(str, c[:4])) + f"-s{c[4]}{c[5]}" + ("-bf16" if c[6] else "-f32"))
def test_strided_depthwise_matches_float64(case):
    """Stride (sh, sw) with pads 1 is the stride-1 'same' convolution taken
    at every sh-th row and sw-th column."""
    n, h, wd, c, sh, sw, dt, want_kernel = case
    lib = _lib()
    f = ctypes.POINTER(ctypes.c_float)
    i = ctypes.c_int
    lib.ppocr_probe_depthwise_strided.argtypes = [f, i, i, i, i, f, f, i, i, i, i, f]
    lib.ppocr_probe_depthwise_strided.restype = i
    lib.ppocr_probe_depthwise_strided_kernel.argtypes = [i, i, i, i, i]
    lib.ppocr_probe_depthwise_strided_kernel.restype = ctypes.c_char_p
    assert lib.ppocr_probe_depthwise_strided_kernel(h, c, sh, sw, dt).decode() == want_kernel
    rng = np.random.default_rng(11 + h + wd + c + sw)
    x = rng.uniform(-1, 1, (n, h, wd, c)).astype(np.float32)
    w = rng.uniform(-0.5, 0.5, (c, 3, 3)).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, c).astype(np.float32)
    ho, wo = (h - 1) // sh + 1, (wd - 1) // sw + 1
    out = np.full((n, ho, wo, c), np.nan, np.float32)
    assert lib.ppocr_probe_depthwise_strided(_ptr(x), n, h, wd, c, _ptr(w), _ptr(b), sh, sw, ACT_HSWISH, dt,
                                             _ptr(out)) == 0
    ref = depthwise_ref(bf16_round(x) if dt else x, w, b, ACT_HSWISH, None)[:, ::sh, ::sw]
    tol = (2.0 ** -8 if dt else 1e-5) * np.abs(ref) + 1e-5
    err = np.abs(out - ref)
    assert np.all(err <= tol), (float(err.max()), np.unravel_index(np.argmax(err - tol), err.shape))
