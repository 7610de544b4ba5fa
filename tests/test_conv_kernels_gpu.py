"""Kernel-level checks of the implicit-GEMM convolution on the GPU.

Every variant launch_conv can pick (1x1 and k x k direct kernels, the gated
direct kernel, the register-staged kernel with its in-gather gate and its
8-byte bf16 loads, split K, bf16 storage) runs through the test harness
libppocr_hip_probe.so on shapes whose M, N and K are not multiples of the
tiles, and is compared with a float64 convolution of the same operands
(the reference conv semantics: zero padding, bias, then the activation,
src/cpu/ops.rs).  Each case first asserts which kernel instance it runs, so
a change in kernel selection cannot silently drop a variant from the test.
"""
import ctypes
import pathlib
import zlib

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
PROBE = ROOT / "ppocr-rs_amd" / "libppocr_hip_probe.so"

ACT_NONE, ACT_RELU, ACT_HSWISH, ACT_SIGMOID = 0, 1, 6, 7


def _lib():
    if not PROBE.exists():
        raise RuntimeError(f"{PROBE} is not built (make -C ppocr-rs_amd)")
    lib = ctypes.CDLL(str(PROBE))
    f = ctypes.POINTER(ctypes.c_float)
    i = ctypes.c_int
    lib.ppocr_probe_conv.argtypes = [f, i, i, i, i, f, f, i, i, i, i, i, i, i, i, i, i, f, i, i, f]
    lib.ppocr_probe_conv.restype = i
    lib.ppocr_probe_conv_kernel.argtypes = [i] * 15 + [ctypes.POINTER(i)]
    lib.ppocr_probe_conv_kernel.restype = ctypes.c_char_p
    return lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def bf16_round(a):
    """Round float32 values to bfloat16 (nearest even; NaN stays NaN),
    returned as float32."""
    x = np.ascontiguousarray(a, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, r)


def act(y, kind):
    if kind == ACT_RELU:
        return np.maximum(y, 0.0)
    if kind == ACT_HSWISH:
        return y * np.clip(y / 6.0 + 0.5, 0.0, 1.0)
    if kind == ACT_SIGMOID:
        return 1.0 / (1.0 + np.exp(-y))
    return y


def conv_ref(x, w, b, stride, pads, kind):
    """float64 NHWC convolution: x [n][h][w][c], w [co][c][kh][kw]."""
    n, h, wd, c = x.shape
    co, _, kh, kw = w.shape
    pt, pl, pb, pr = pads
    xp = np.zeros((n, h + pt + pb, wd + pl + pr, c))
    xp[:, pt:pt + h, pl:pl + wd, :] = x
    ho = (h + pt + pb - kh) // stride[0] + 1
    wo = (wd + pl + pr - kw) // stride[1] + 1
    y = np.zeros((n, ho, wo, co))
    for ky in range(kh):
        for kx in range(kw):
            patch = xp[:, ky:ky + stride[0] * (ho - 1) + 1:stride[0], kx:kx + stride[1] * (wo - 1) + 1:stride[1], :]
            y += patch @ w[:, :, ky, kx].T.astype(np.float64)
    if b is not None:
        y += b
    return act(y, kind)


# (name, n, h, w, c, co, (kh, kw), (sh, sw), (pt, pl, pb, pr), gated, splits, dt, act, expected kernel)
# Layers of fewer than 1024 64x64 tiles take 64-row tiles of 32 columns; the
# "64x64" cases are sized past that (>= 1024 tiles).
CASES = [
    ("1x1 M/N tails", 2, 7, 9, 64, 96, (1, 1), (1, 1), (0, 0, 0, 0), False, 1, 0, ACT_RELU, "conv_gemm<64x32,1x1>"),
    ("1x1 M/N tails 64x64", 1, 181, 183, 64, 96, (1, 1), (1, 1), (0, 0, 0, 0), False, 1, 0, ACT_RELU,
     "conv_gemm<64x64,1x1>"),
    ("3x3 K tail", 1, 11, 13, 20, 24, (3, 3), (1, 1), (1, 1, 1, 1), False, 1, 0, ACT_HSWISH, "conv_gemm<64x32>"),
    ("3x3 stride 2", 2, 12, 10, 16, 64, (3, 3), (2, 2), (1, 1, 1, 1), False, 1, 0, ACT_NONE, "conv_gemm<64x32>"),
    ("3x3 stride 2 64x64", 1, 365, 363, 16, 96, (3, 3), (2, 2), (1, 1, 1, 1), False, 1, 0, ACT_NONE,
     "conv_gemm<64x64>"),
    ("7x1 asymmetric", 1, 9, 6, 8, 24, (7, 1), (1, 1), (3, 0, 3, 0), False, 1, 0, ACT_RELU, "conv_gemm<64x32>"),
    ("1x1 narrow Co", 1, 5, 6, 12, 10, (1, 1), (1, 1), (0, 0, 0, 0), False, 1, 0, ACT_SIGMOID, "conv_gemm<64x16,1x1>"),
    ("1x1 narrow Co, 512 row tiles", 1, 512, 256, 16, 12, (1, 1), (1, 1), (0, 0, 0, 0), False, 1, 0, ACT_RELU,
     "conv_gemm<256x16,1x1>"),
    ("3x3 narrow Co", 2, 13, 11, 8, 12, (3, 3), (1, 1), (1, 1, 1, 1), False, 1, 0, ACT_HSWISH, "conv_gemm<64x16>"),
    ("1x1 Co 24, 512 row tiles", 1, 256, 256, 8, 24, (1, 1), (1, 1), (0, 0, 0, 0), False, 1, 0, ACT_NONE,
     "conv_gemm<128x32,1x1>"),
    ("gated 1x1 direct", 3, 8, 10, 64, 64, (1, 1), (1, 1), (0, 0, 0, 0), True, 1, 0, ACT_RELU,
     "conv_gemm<64x32,1x1,gate>"),
    ("gated 1x1 direct 64x64", 8, 64, 72, 64, 128, (1, 1), (1, 1), (0, 0, 0, 0), True, 1, 0, ACT_RELU,
     "conv_gemm<64x64,1x1,gate>"),
    ("gated 1x1 small images", 5, 3, 5, 64, 64, (1, 1), (1, 1), (0, 0, 0, 0), True, 1, 0, ACT_NONE,
     "conv_gemm<64x32,1x1,reg>"),
    ("gated 1x1 small images 64x64", 2400, 3, 5, 64, 128, (1, 1), (1, 1), (0, 0, 0, 0), True, 1, 0, ACT_NONE,
     "conv_gemm<64x64,1x1,reg>"),
    ("split K 1x1", 1, 5, 7, 256, 64, (1, 1), (1, 1), (0, 0, 0, 0), False, 4, 0, ACT_RELU, "conv_gemm<64x32,1x1>"),
    ("split K 1x1 64x64", 1, 181, 183, 256, 96, (1, 1), (1, 1), (0, 0, 0, 0), False, 3, 0, ACT_RELU,
     "conv_gemm<64x64,1x1>"),
    ("split K 3x3 uneven", 2, 6, 5, 32, 32, (3, 3), (1, 1), (1, 1, 1, 1), False, 5, 0, ACT_HSWISH,
     "conv_gemm<64x32>"),
    ("split K gated", 2, 6, 12, 128, 64, (1, 1), (1, 1), (0, 0, 0, 0), True, 3, 0, ACT_NONE,
     "conv_gemm<64x32,1x1,gate>"),
    ("bf16 1x1", 2, 9, 7, 64, 96, (1, 1), (1, 1), (0, 0, 0, 0), False, 1, 1, ACT_RELU, "conv_gemm_bf16<64x32,1x1>"),
    ("bf16 1x1 64x64", 1, 181, 183, 64, 96, (1, 1), (1, 1), (0, 0, 0, 0), False, 1, 1, ACT_RELU,
     "conv_gemm_bf16<64x64,1x1>"),
    ("bf16 3x3", 1, 10, 12, 32, 64, (3, 3), (1, 1), (1, 1, 1, 1), False, 1, 1, ACT_NONE, "conv_gemm_bf16<64x32>"),
    ("bf16 3x3 64x64", 1, 181, 183, 32, 96, (3, 3), (1, 1), (1, 1, 1, 1), False, 1, 1, ACT_NONE,
     "conv_gemm_bf16<64x64>"),
    ("bf16 C % 8 = 4", 1, 8, 9, 12, 48, (3, 3), (1, 1), (1, 1, 1, 1), False, 1, 1, ACT_RELU,
     "conv_gemm_bf16<64x32,reg4>"),
    ("bf16 C % 8 = 4 64x64", 1, 181, 183, 12, 96, (3, 3), (1, 1), (1, 1, 1, 1), False, 1, 1, ACT_RELU,
     "conv_gemm_bf16<64x64,reg4>"),
    ("bf16 gated", 2, 8, 10, 64, 64, (1, 1), (1, 1), (0, 0, 0, 0), True, 1, 1, ACT_NONE,
     "conv_gemm_bf16<64x32,1x1,reg>"),
    ("bf16 gated 64x64", 2400, 3, 5, 64, 128, (1, 1), (1, 1), (0, 0, 0, 0), True, 1, 1, ACT_NONE,
     "conv_gemm_bf16<64x64,1x1,reg>"),
    ("bf16 split K", 1, 7, 5, 256, 64, (1, 1), (1, 1), (0, 0, 0, 0), False, 2, 1, ACT_RELU,
     "conv_gemm_bf16<64x32,1x1>"),
    ("bf16 128-byte rows", 5, 37, 41, 776, 520, (1, 1), (1, 1), (0, 0, 0, 0), False, 1, 1, ACT_HSWISH,
     "conv_gemm_bf16<64x64,1x1,r128>"),
    ("bf16 3x3 128-byte rows", 17, 19, 23, 320, 520, (3, 3), (1, 1), (1, 1, 1, 1), False, 1, 1, ACT_RELU,
     "conv_gemm_bf16<64x64,r128>"),
    ("bf16 3x3 s2 128-byte rows", 208, 21, 17, 128, 200, (3, 3), (2, 2), (1, 1, 0, 0), False, 1, 1, ACT_NONE,
     "conv_gemm_bf16<64x64,r128>"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_conv_variant_matches_float64(case):
    name, n, h, w, c, co, (kh, kw), (sh, sw), pads, gated, splits, dt, kind, want_kernel = case
    lib = _lib()
    kernel = lib.ppocr_probe_conv_kernel(n, h, w, c, co, kh, kw, sh, sw, *pads, int(gated), dt, None).decode()
    assert kernel == want_kernel, f"{name}: runs {kernel}"

    rng = np.random.default_rng(zlib.crc32(name.encode()))
    x = rng.standard_normal((n, h, w, c)).astype(np.float32)
    wt = (rng.standard_normal((co, c, kh, kw)) / np.sqrt(c * kh * kw)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32) * 0.1
    g = rng.uniform(0.0, 1.0, (n, c)).astype(np.float32) if gated else None
    ho = (h + pads[0] + pads[2] - kh) // sh + 1
    wo = (w + pads[1] + pads[3] - kw) // sw + 1
    out = np.empty((n, ho, wo, co), dtype=np.float32)
    rc = lib.ppocr_probe_conv(_ptr(x), n, h, w, c, _ptr(wt), _ptr(b), co, kh, kw, sh, sw, *pads, kind, _ptr(g),
                              splits, dt, _ptr(out))
    assert rc == 0

    if dt == 1:
        # The kernel multiplies bf16 operands (and, gated, bf16(x * g)) with
        # fp32 accumulation and stores the result in bf16.
        xs = bf16_round(x)
        if gated:
            xs = bf16_round(xs * g[:, None, None, :])
        ref = conv_ref(xs.astype(np.float64), bf16_round(wt).astype(np.float64), b, (sh, sw), pads, kind)
        tol = 1e-3 + 8e-3 * np.abs(ref)
    else:
        xs = x * g[:, None, None, :] if gated else x
        ref = conv_ref(xs.astype(np.float64), wt.astype(np.float64), b, (sh, sw), pads, kind)
        tol = 1e-4 + 1e-5 * np.abs(ref)
    err = np.abs(out - ref)
    assert np.all(err <= tol), f"{name} ({kernel}): max abs diff {err.max():.3e}"


@pytest.mark.gpu
def test_split_k_agrees_with_unsplit():
    """The same layer with 1, 2 and 7 K splits: results agree to fp32 rounding."""
    lib = _lib()
    rng = np.random.default_rng(3)
    n, h, w, c, co = 1, 6, 9, 192, 64
    x = rng.standard_normal((n, h, w, c)).astype(np.float32)
    wt = (rng.standard_normal((co, c, 3, 3)) / np.sqrt(9 * c)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32)
    outs = []
    for splits in (1, 2, 7):
        out = np.empty((n, h, w, co), dtype=np.float32)
        assert lib.ppocr_probe_conv(_ptr(x), n, h, w, c, _ptr(wt), _ptr(b), co, 3, 3, 1, 1, 1, 1, 1, 1, ACT_NONE,
                                    None, splits, 0, _ptr(out)) == 0
        outs.append(out)
    for o in outs[1:]:
        assert np.max(np.abs(o - outs[0])) <= 1e-4


# Fused pointwise pair (pair_gemm.hip): out = w2 GELU(w1 x' + b1) + b2
# (+ x'), x' = x * gate[image], against float64 with the exact-erf GELU (the
# kernel's A-S erf differs by < 1.5e-7).  Rows not a multiple of the 32-pixel
# tile, tiles straddling images, 16-channel multiples from 16 to 192.
PAIR_CASES = [
    # name, rows, pixels per image, C, Co, gate, residual
    ("tiny stage 1 residual gated", 1000, 400, 32, 32, True, True),
    ("plain, one tile", 17, 17, 16, 16, False, False),
    ("widen, no residual", 333, 111, 48, 96, False, False),
    ("residual", 259, 259, 64, 64, False, True),
    ("gated, narrow", 70, 23, 96, 48, True, False),
    ("widest", 95, 45, 192, 192, True, True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,m,hw,c,co,gated,residual", PAIR_CASES, ids=[c[0] for c in PAIR_CASES])
def test_pointwise_pair_matches_float64(name, m, hw, c, co, gated, residual):
    from scipy.special import erf

    lib = _lib()
    f = ctypes.POINTER(ctypes.c_float)
    i = ctypes.c_int
    lib.ppocr_probe_pointwise_pair.argtypes = [f, i, i, i, f, f, f, i, f, f, i, i, f]
    lib.ppocr_probe_pointwise_pair.restype = i
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    h2 = 2 * c
    x = rng.standard_normal((m, c)).astype(np.float32)
    n = (m + hw - 1) // hw
    gate = rng.uniform(0, 1, (n, c)).astype(np.float32) if gated else None
    w1 = (rng.standard_normal((h2, c)) / np.sqrt(c)).astype(np.float32)
    b1 = rng.standard_normal(h2).astype(np.float32) * 0.1
    w2 = (rng.standard_normal((co, h2)) / np.sqrt(h2)).astype(np.float32)
    b2 = rng.standard_normal(co).astype(np.float32) * 0.1
    out = np.empty((m, co), np.float32)
    rc = lib.ppocr_probe_pointwise_pair(_ptr(x), m, hw, c, _ptr(gate), _ptr(w1), _ptr(b1), h2, _ptr(w2), _ptr(b2), co,
                                        int(residual), _ptr(out))
    assert rc == 0
    xg = x.astype(np.float64)
    if gated:
        xg = (x * gate[np.arange(m) // hw]).astype(np.float64)  # x * g rounded to fp32, as the kernel forms it
    h = xg @ w1.T.astype(np.float64) + b1
    h = 0.5 * h * (1.0 + erf(h / np.sqrt(2.0)))
    want = h @ w2.T.astype(np.float64) + b2
    if residual:
        want = want + xg
    err = np.abs(out - want)
    assert np.all(err <= 1e-4 + 1e-5 * np.abs(want)), f"max err {err.max()}"


# The fused bf16 pair (C -> 2C -> C) against the unfused bf16 plan's own
# launches on the same device data, which it must equal bit for bit (same
# MFMA instruction, k order and rounding points), and against a float64
# evaluation with the plan's bf16 roundings (x, x * g, the GELU output and
# the result rounded to bf16): within one bf16 ulp of the larger magnitude
# (the final rounding, which can also cross a power of two) plus 2e-3 for
# GELU outputs near a rounding tie that round the other way in float64.  Rows not a multiple
# of the 16- or 32-row wave blocks, blocks straddling images, and row counts
# on both sides of the 32-row threshold (a block per wave of 256 CUs x 8
# waves: 65536 rows).
PAIR_BF16_CASES = [
    # name, rows, pixels per image, C, gate, residual, rows per wave block
    ("C128 gated residual", 3000, 700, 128, True, True, 16),
    ("C128 plain, one block", 9, 9, 128, False, False, 16),
    ("C128 residual, 32-row blocks", 66001, 66001, 128, False, True, 32),
    ("C128 gated, 32-row blocks", 70000, 9999, 128, True, False, 32),
    ("C96 gated residual", 1999, 333, 96, True, True, 16),
    ("C64 residual", 4097, 4097, 64, False, True, 16),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,m,hw,c,gated,residual,rows", PAIR_BF16_CASES, ids=[c[0] for c in PAIR_BF16_CASES])
def test_pair_bf16_equals_unfused_bf16_plan(name, m, hw, c, gated, residual, rows):
    from scipy.special import erf

    lib = _lib()
    f = ctypes.POINTER(ctypes.c_float)
    i = ctypes.c_int
    lib.ppocr_probe_pair_bf16.argtypes = [f, i, i, i, f, f, f, f, f, i, f, f, ctypes.c_char_p, ctypes.c_size_t]
    lib.ppocr_probe_pair_bf16.restype = i
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    x = rng.standard_normal((m, c)).astype(np.float32)
    n = (m + hw - 1) // hw
    gate = rng.uniform(0, 1, (n, c)).astype(np.float32) if gated else None
    w1 = (rng.standard_normal((2 * c, c)) / np.sqrt(c)).astype(np.float32)
    b1 = rng.standard_normal(2 * c).astype(np.float32) * 0.1
    w2 = (rng.standard_normal((c, 2 * c)) / np.sqrt(2 * c)).astype(np.float32)
    b2 = rng.standard_normal(c).astype(np.float32) * 0.1
    fused = np.full((m, c), np.nan, np.float32)
    unfused = np.full((m, c), np.nan, np.float32)
    kernel = ctypes.create_string_buffer(64)
    rc = lib.ppocr_probe_pair_bf16(_ptr(x), m, hw, c, _ptr(gate), _ptr(w1), _ptr(b1), _ptr(w2), _ptr(b2),
                                   int(residual), _ptr(fused), _ptr(unfused), kernel, 64)
    assert rc == 0
    want_name = f"pair_bf16<{c},{rows}" + (",gate" if gated else "") + (",res" if residual else "") + ">"
    assert kernel.value.decode() == want_name
    diff = np.flatnonzero(fused.view(np.uint32) != unfused.view(np.uint32))
    assert diff.size == 0, f"{diff.size} outputs differ from the unfused plan, first at {np.unravel_index(diff[0], fused.shape)}"
    xb = bf16_round(x)
    xg = bf16_round(xb * gate[np.arange(m) // hw]) if gated else xb
    h = xg.astype(np.float64) @ bf16_round(w1).T.astype(np.float64) + b1
    h = bf16_round((0.5 * h * (1.0 + erf(h / np.sqrt(2.0)))).astype(np.float32))
    want = h.astype(np.float64) @ bf16_round(w2).T.astype(np.float64) + b2
    if residual:
        want = want + xg
    err = np.abs(fused - want)
    assert np.all(err <= 2.0 ** -7 * np.maximum(np.abs(want), np.abs(fused)) + 2e-3), f"max err {err.max()}"


# (name, m, c, co, partial rows, residual): one image whose SE gate the pair
# kernel forms from partial channel sums, one to three rounds of eight rows
# per lane.
PAIR_SE_CASES = [
    ("C32, 250 partial rows, residual", 900, 32, 32, 250, True),
    ("C48, 84 partial rows", 333, 48, 96, 84, False),
    ("C64, 128 partial rows, residual", 1000, 64, 64, 128, True),
    ("C64, one partial row", 40, 64, 64, 1, False),
    ("C32, 600 partial rows in three rounds", 2000, 32, 32, 600, True),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,m,c,co,P,residual", PAIR_SE_CASES, ids=[c[0] for c in PAIR_SE_CASES])
def test_pointwise_pair_forms_se_gate(name, m, c, co, P, residual):
    """The pair kernel's SE prologue: channel means from P partial sums, the
    two small convs (ReLU, then hard-sigmoid(x/6 + 0.5)), x * gate, then the
    pair, against float64 (the gate's sums run in another order than the
    gate kernel's, within fp32 rounding)."""
    from scipy.special import erf

    lib = _lib()
    f = ctypes.POINTER(ctypes.c_float)
    i = ctypes.c_int
    lib.ppocr_probe_pointwise_pair_se.argtypes = [f, i, i, f, i, f, f, i, f, f, i, f, f, i, f, f, i, i, f]
    lib.ppocr_probe_pointwise_pair_se.restype = i
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    h2, cr = 2 * c, c // 4
    x = rng.standard_normal((m, c)).astype(np.float32)
    part = rng.standard_normal((P, c)).astype(np.float32) * np.float32(m / P)
    sw1 = (rng.standard_normal((cr, c)) / np.sqrt(c)).astype(np.float32)
    sb1 = rng.standard_normal(cr).astype(np.float32) * 0.1
    sw2 = (rng.standard_normal((c, cr)) / np.sqrt(cr)).astype(np.float32)
    sb2 = rng.standard_normal(c).astype(np.float32) * 0.1
    w1 = (rng.standard_normal((h2, c)) / np.sqrt(c)).astype(np.float32)
    b1 = rng.standard_normal(h2).astype(np.float32) * 0.1
    w2 = (rng.standard_normal((co, h2)) / np.sqrt(h2)).astype(np.float32)
    b2 = rng.standard_normal(co).astype(np.float32) * 0.1
    out = np.empty((m, co), np.float32)
    ACT_HSIG6 = 4
    rc = lib.ppocr_probe_pointwise_pair_se(_ptr(x), m, c, _ptr(part), P, _ptr(sw1), _ptr(sb1), cr, _ptr(sw2),
                                           _ptr(sb2), ACT_HSIG6, _ptr(w1), _ptr(b1), h2, _ptr(w2), _ptr(b2), co,
                                           int(residual), _ptr(out))
    assert rc == 0
    mean = part.astype(np.float64).sum(axis=0) / m
    hid = np.maximum(sw1.astype(np.float64) @ mean + sb1, 0.0)
    gate = np.clip((sw2.astype(np.float64) @ hid + sb2) / 6.0 + 0.5, 0.0, 1.0)
    xg = x.astype(np.float64) * gate
    h = xg @ w1.T.astype(np.float64) + b1
    h = 0.5 * h * (1.0 + erf(h / np.sqrt(2.0)))
    want = h @ w2.T.astype(np.float64) + b2
    if residual:
        want = want + xg
    err = np.abs(out - want)
    assert np.all(err <= 1e-4 + 1e-5 * np.abs(want)), f"max err {err.max()}"


# (name, n, h, w, c, stride, co, residual): maps whose pixel count is not a
# multiple of the 32-pixel tile, strides 1 and 2, a tile spanning two images.
PAIR_DW_CASES = [
    ("s1 residual", 2, 13, 11, 32, 1, 32, True),
    ("s1 plain", 1, 9, 20, 16, 1, 48, False),
    ("s2", 2, 15, 18, 64, 2, 64, False),
    ("s2 odd", 1, 7, 9, 16, 2, 32, False),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,n,h,w,c,stride,co,residual", PAIR_DW_CASES, ids=[c[0] for c in PAIR_DW_CASES])
def test_pointwise_pair_depthwise_prologue_matches_float64(name, n, h, w, c, stride, co, residual):
    from scipy.special import erf

    lib = _lib()
    f = ctypes.POINTER(ctypes.c_float)
    i = ctypes.c_int
    lib.ppocr_probe_pointwise_pair_dw.argtypes = [f, i, i, i, i, f, f, i, i, f, f, i, f, f, i, i, f]
    lib.ppocr_probe_pointwise_pair_dw.restype = i
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    h2 = 2 * c
    x = rng.standard_normal((n, h, w, c)).astype(np.float32)
    dw = (rng.standard_normal((9, c)) / 3).astype(np.float32)
    dwb = rng.standard_normal(c).astype(np.float32) * 0.1
    w1 = (rng.standard_normal((h2, c)) / np.sqrt(c)).astype(np.float32)
    b1 = rng.standard_normal(h2).astype(np.float32) * 0.1
    w2 = (rng.standard_normal((co, h2)) / np.sqrt(h2)).astype(np.float32)
    b2 = rng.standard_normal(co).astype(np.float32) * 0.1
    ho, wo = (h - 1) // stride + 1, (w - 1) // stride + 1
    out = np.empty((n, ho, wo, co), np.float32)
    rc = lib.ppocr_probe_pointwise_pair_dw(_ptr(x), n, h, w, c, _ptr(dw), _ptr(dwb), stride, stride, _ptr(w1),
                                           _ptr(b1), h2, _ptr(w2), _ptr(b2), co, int(residual), _ptr(out))
    assert rc == 0
    # float64 3x3 depthwise, pads 1, then the pair.
    xp = np.pad(x.astype(np.float64), ((0, 0), (1, 1), (1, 1), (0, 0)))
    t = np.zeros((n, ho, wo, c))
    for ky in range(3):
        for kx in range(3):
            t += xp[:, ky:ky + stride * (ho - 1) + 1:stride, kx:kx + stride * (wo - 1) + 1:stride, :] * dw[ky * 3 + kx]
    t += dwb
    hid = t @ w1.T.astype(np.float64) + b1
    hid = 0.5 * hid * (1.0 + erf(hid / np.sqrt(2.0)))
    want = hid @ w2.T.astype(np.float64) + b2
    if residual:
        want = want + t
    err = np.abs(out - want)
    assert np.all(err <= 1e-4 + 1e-5 * np.abs(want)), f"max err {err.max()}"


# (name, n, h, w, c, co, rep): upsample-on-write convs; K <= 64 writes one
# replica per workgroup layer, wider K all replicas per workgroup.
REP_CASES = [
    ("rep8 K32", 2, 5, 7, 32, 64, 8),
    ("rep4 K32", 1, 13, 23, 32, 64, 4),
    ("rep2 K32 tails", 1, 9, 11, 32, 48, 2),
    ("rep4 K96", 1, 6, 9, 96, 64, 4),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,n,h,w,c,co,rep", REP_CASES, ids=[c[0] for c in REP_CASES])
def test_upsample_on_write_matches_float64(name, n, h, w, c, co, rep):
    lib = _lib()
    f = ctypes.POINTER(ctypes.c_float)
    i = ctypes.c_int
    lib.ppocr_probe_conv_rep.argtypes = [f, i, i, i, i, f, f, i, i, f, i, f]
    lib.ppocr_probe_conv_rep.restype = i
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    x = rng.standard_normal((n, h, w, c)).astype(np.float32)
    wt = (rng.standard_normal((co, c)) / np.sqrt(c)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32) * 0.1
    res = rng.standard_normal((n, h, w, co)).astype(np.float32)
    out = np.full((n, h * rep, w * rep, co), np.nan, np.float32)
    assert lib.ppocr_probe_conv_rep(_ptr(x), n, h, w, c, _ptr(wt), _ptr(b), co, ACT_RELU, _ptr(res), rep,
                                    _ptr(out)) == 0
    y = res + np.maximum(x.astype(np.float64) @ wt.T.astype(np.float64) + b, 0.0)
    want = np.repeat(np.repeat(y, rep, axis=1), rep, axis=2)
    assert np.all(np.isfinite(out)), "an output block was not written"
    err = np.abs(out - want)
    assert np.all(err <= 1e-4 + 1e-5 * np.abs(want)), f"{name}: max abs diff {err.max():.3e}"


# Wide-tile bf16 1x1 kernel (256x256 tiles of 32x32x16 MFMAs): M, N and K
# tails, plain and gated residual, and a layer just below its K threshold;
# grids of fewer and of more tiles than the persistent workgroups.
# (name, n, h, w, c, co, act, residual: 0 none / 1 plain / 2 gated, fp32 output, kernel)
ACT_GELU = 2
WIDE_CASES = [
    ("wide M/N/K tails", 2, 65, 127, 520, 520, ACT_HSWISH, 0, False, "conv_gemm_bf16<256x256,1x1>"),
    # bf16 outputs leave the wide kernel 8 columns at a time: Co % 8 = 4 runs
    # on the direct kernel.
    ("wide shape, Co % 8 = 4", 2, 65, 127, 520, 516, ACT_HSWISH, 0, False, "conv_gemm_bf16<64x64,1x1>"),
    ("wide residual", 1, 130, 127, 512, 512, ACT_NONE, 1, False, "conv_gemm_bf16<256x256,1x1>"),
    ("wide gated residual", 4, 33, 128, 768, 264, ACT_GELU, 2, False, "conv_gemm_bf16<256x256,1x1>"),
    ("K below threshold", 2, 65, 127, 256, 516, ACT_RELU, 1, False, "conv_gemm_bf16<64x64,1x1>"),
    # The classifier form: fp32 logits, Co % 4 == 2 (float2 stores), short K.
    ("wide fp32 out, Co % 4 = 2", 1, 61, 110, 200, 1030, ACT_NONE, 0, True, "conv_gemm_bf16<256x256,1x1>"),
    # More tiles than compute units: each persistent workgroup walks several
    # tiles, the next tile's first K slice loading during the epilogue.
    ("wide persistent, 432 tiles", 4, 96, 96, 520, 520, ACT_GELU, 0, False, "conv_gemm_bf16<256x256,1x1>"),
    ("wide persistent residual, 354 tiles", 3, 100, 100, 512, 768, ACT_NONE, 1, False, "conv_gemm_bf16<256x256,1x1>"),
    ("wide persistent gated residual", 8, 64, 80, 576, 512, ACT_RELU, 2, False, "conv_gemm_bf16<256x256,1x1>"),
    ("wide persistent fp32 out", 2, 100, 160, 192, 2050, ACT_NONE, 0, True, "conv_gemm_bf16<256x256,1x1>"),
]


@pytest.mark.gpu
@pytest.mark.parametrize("name,n,h,w,c,co,kind,residual,f32out,want_kernel", WIDE_CASES,
                         ids=[c[0] for c in WIDE_CASES])
def test_wide_bf16_1x1_matches_float64(name, n, h, w, c, co, kind, residual, f32out, want_kernel):
    from scipy.special import erf

    lib = _lib()
    f = ctypes.POINTER(ctypes.c_float)
    i = ctypes.c_int
    lib.ppocr_probe_conv1x1_res.argtypes = [f, i, i, i, i, f, f, i, i, f, f, i, i, f, ctypes.POINTER(ctypes.c_char_p)]
    lib.ppocr_probe_conv1x1_res.restype = i
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    x = rng.standard_normal((n, h, w, c)).astype(np.float32)
    wt = (rng.standard_normal((co, c)) / np.sqrt(c)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32) * 0.1
    res = rng.standard_normal((n, h, w, co)).astype(np.float32) if residual else None
    rg = rng.uniform(0.0, 1.0, (n, co)).astype(np.float32) if residual == 2 else None
    out = np.empty((n, h, w, co), dtype=np.float32)
    kernel = ctypes.c_char_p()
    assert lib.ppocr_probe_conv1x1_res(_ptr(x), n, h, w, c, _ptr(wt), _ptr(b), co, kind, _ptr(res), _ptr(rg), 1,
                                       int(f32out), _ptr(out), ctypes.byref(kernel)) == 0
    assert kernel.value.decode() == want_kernel, f"{name}: runs {kernel.value.decode()}"

    y = bf16_round(x).astype(np.float64).reshape(-1, c) @ bf16_round(wt).astype(np.float64).T + b
    if kind == ACT_GELU:
        y = 0.5 * y * (1.0 + erf(y / np.sqrt(2.0)))
    else:
        y = act(y, kind)
    y = y.reshape(n, h, w, co)
    if residual:
        r = bf16_round(res).astype(np.float64)
        if residual == 2:
            r = r * rg[:, None, None, :]
        y = y + r
    # bf16 storage rounds the output (2^-9 relative); fp32 logits keep only
    # the fp32 accumulation error.
    tol = 1e-3 + (1e-5 if f32out else 8e-3) * np.abs(y)
    err = np.abs(out - y)
    assert np.all(err <= tol), f"{name} ({want_kernel}): max abs diff {err.max():.3e}"


# (name, h, w, c, co, (kh, kw), pads, gated, dt, act, expected kernel, rows per tile row block or 0)
SE_CASES = [
    ("se sums 64x64 fp32", 256, 260, 64, 64, (1, 1), (0, 0, 0, 0), False, 0, ACT_RELU, "conv_gemm<64x64,1x1>", 2),
    ("se sums 64x32 fp32, 64 columns", 23, 29, 64, 64, (1, 1), (0, 0, 0, 0), False, 0, ACT_RELU, "conv_gemm<64x32,1x1>",
     4),
    ("se sums 64x16", 19, 37, 32, 16, (1, 1), (0, 0, 0, 0), False, 0, ACT_NONE, "conv_gemm<64x16,1x1>", 4),
    ("se sums 64x32", 17, 21, 32, 24, (1, 1), (0, 0, 0, 0), False, 0, ACT_HSWISH, "conv_gemm<64x32,1x1>", 4),
    ("no se sums: 3x3", 17, 21, 32, 24, (3, 3), (1, 1, 1, 1), False, 0, ACT_HSWISH, "conv_gemm<64x32>", 0),
    ("no se sums: bf16 (LDS epilogue)", 17, 21, 32, 24, (3, 3), (1, 1, 1, 1), False, 1, ACT_HSWISH,
     "conv_gemm_bf16<64x32>", 0),
    ("no se sums: gated", 13, 23, 64, 96, (1, 1), (0, 0, 0, 0), True, 0, ACT_NONE, "conv_gemm<64x32,1x1,gate>", 0),
    ("no se sums: Co % 4 = 2", 9, 11, 16, 6, (1, 1), (0, 0, 0, 0), False, 0, ACT_NONE, "conv_gemm<64x16,1x1>", 0),
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", SE_CASES, ids=[c[0] for c in SE_CASES])
def test_conv_se_channel_sums(case):
    """The squeeze-excitation channel sums a single-image fp32 1x1 conv
    leaves in its register epilogue: summed over their rows they equal the
    column sums of the output the conv stored (each row holds one wave's rows
    of one tile), and the output itself still matches the float64
    convolution.  Other layers report no sums."""
    name, h, w, c, co, (kh, kw), pads, gated, dt, kind, want_kernel, per_block = case
    lib = _lib()
    f = ctypes.POINTER(ctypes.c_float)
    i = ctypes.c_int
    lib.ppocr_probe_conv_se.argtypes = [f, i, i, i, f, f, i, i, i, i, i, i, i, i, i, i, f, i, f,
                                        ctypes.POINTER(i), f]
    lib.ppocr_probe_conv_se.restype = i
    kernel = lib.ppocr_probe_conv_kernel(1, h, w, c, co, kh, kw, 1, 1, *pads, int(gated), dt, None).decode()
    assert kernel == want_kernel, f"{name}: runs {kernel}"

    rng = np.random.default_rng(zlib.crc32(name.encode()))
    x = rng.standard_normal((1, h, w, c)).astype(np.float32)
    wt = (rng.standard_normal((co, c, kh, kw)) / np.sqrt(c * kh * kw)).astype(np.float32)
    b = rng.standard_normal(co).astype(np.float32) * 0.1
    g = rng.uniform(0.0, 1.0, (1, c)).astype(np.float32) if gated else None
    ho = h + pads[0] + pads[2] - kh + 1
    wo = w + pads[1] + pads[3] - kw + 1
    out = np.empty((1, ho, wo, co), dtype=np.float32)
    cap = (ho * wo + 15) // 16 + 4
    part = np.full((cap, co), np.nan, dtype=np.float32)
    rows = ctypes.c_int(-1)
    rc = lib.ppocr_probe_conv_se(_ptr(x), h, w, c, _ptr(wt), _ptr(b), co, kh, kw, 1, 1, *pads, kind, _ptr(g), dt,
                                 _ptr(out), ctypes.byref(rows), _ptr(part))
    assert rc == 0
    bm = int(want_kernel.split("<")[1].split("x")[0])
    assert rows.value == ((ho * wo + bm - 1) // bm) * per_block, f"{name}: {rows.value} rows"

    if dt == 1:
        xs = bf16_round(x)
        ref = conv_ref(xs.astype(np.float64), bf16_round(wt).astype(np.float64), b, (1, 1), pads, kind)
        tol = 1e-3 + 8e-3 * np.abs(ref)
    else:
        xs = x * g[:, None, None, :] if gated else x
        ref = conv_ref(xs.astype(np.float64), wt.astype(np.float64), b, (1, 1), pads, kind)
        tol = 1e-4 + 1e-5 * np.abs(ref)
    assert np.all(np.abs(out - ref) <= tol), f"{name}: output differs"
    if rows.value == 0:
        return
    sums = part[:rows.value].astype(np.float64).sum(axis=0)
    want = out.astype(np.float64).sum(axis=(0, 1, 2))
    scale = np.abs(out).astype(np.float64).sum(axis=(0, 1, 2))
    assert np.all(np.abs(sums - want) <= 1e-5 * scale + 1e-6), f"{name}: sums differ by {np.abs(sums - want).max():.3e}"
