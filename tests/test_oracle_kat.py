"""Pins the CPU oracle against the reference's own known-answer tests and
against closed forms, so a plausible restatement mistake (a dropped term, a
wrong index, a transposed operand, a fused instead of a two-step rounding)
fails here.  Each test names the reference test or formula it reproduces.
"""

import math

import numpy as np
import pytest

import oracle

F32 = np.float32


def test_erf_matches_known_values():
    # src/cpu/kernels/mod.rs:2410-2414
    assert abs(oracle.erf(0.0)) < 1e-6
    assert abs(oracle.erf(1.0) - 0.8427008) < 2e-7
    assert abs(oracle.erf(-2.0) + 0.9953223) < 2e-7


def test_gelu_is_exact_erf_gelu_within_the_as_bound():
    # A-S 7.1.26 has |error| <= 1.5e-7, so GELU differs from the exact-erf
    # GELU by <= 0.5 |x| 1.5e-7 (+ rounding); a wrong coefficient breaks this.
    for i in range(1025):
        x = i * (16.0 / 1024.0) - 8.0
        exact = 0.5 * x * (1.0 + math.erf(x / math.sqrt(2.0)))
        assert abs(oracle.act("gelu", x) - exact) <= 0.5 * abs(x) * 1.6e-7 + 2e-6


@pytest.mark.parametrize("x", [-7.5, -3.0, -0.4, 0.0, 0.3, 2.9, 3.1, 6.5])
def test_activation_closed_forms(x):
    # UnaryOperation::apply (src/cpu/kernels/mod.rs:2376-2390)
    xf = float(F32(x))
    assert oracle.act("relu", xf) == max(xf, 0.0)
    assert oracle.act("silu", xf) == pytest.approx(xf / (1 + math.exp(-xf)), rel=1e-6, abs=1e-7)
    assert oracle.act("sigmoid", xf) == pytest.approx(1 / (1 + math.exp(-xf)), rel=1e-6, abs=1e-7)
    assert oracle.act("hswish", xf) == pytest.approx(xf * min(max(xf / 6 + 0.5, 0), 1), rel=1e-6, abs=1e-7)
    assert oracle.act("hsig6", xf) == pytest.approx(min(max(xf / 6 + 0.5, 0), 1), abs=1e-7)
    assert oracle.act("hsig5", xf) == pytest.approx(min(max(xf * 0.2 + 0.5, 0), 1), abs=1e-7)


def test_linear_fuses_bias_and_softmax():
    # src/cpu/backend.rs:1402-1415
    w = np.array([[1.0, 0.0, -1.0], [0.0, 1.0, 1.0]], F32)
    b = np.array([0.5, -0.5], F32)
    x = np.array([[2.0, 3.0, 1.0]], F32)
    assert oracle.linear(x, w, b).tolist() == [[1.5, 3.5]]
    p = oracle.linear(x, w, b, softmax=True)[0]
    assert abs(p[0] + p[1] - 1.0) < 1e-6 and p[1] > p[0]


def test_linear_matches_matmul_with_leading_dimensions():
    # src/cpu/backend.rs:1417-1447
    w = np.array([1.0, 0.0, -1.0, 0.5, -0.25, 2.0, 1.5, 0.75, -0.5, -1.0, 1.0, 0.25], F32).reshape(4, 3)
    b = np.array([0.5, -0.25, 1.0, -0.75], F32)
    x = ((np.arange(36) * 7 % 19).astype(F32) - 9.0) / 5.0
    x = x.reshape(2, 3, 2, 3)
    expected = x.astype(np.float64) @ w.T.astype(np.float64) + b
    actual = oracle.linear(x, w, b)
    assert actual.shape == (2, 3, 2, 4)
    assert np.all(np.abs(actual - expected) <= 3e-5 * (1 + np.abs(expected)))
    e = np.exp(expected - expected.max(-1, keepdims=True))
    e /= e.sum(-1, keepdims=True)
    assert np.all(np.abs(oracle.linear(x, w, b, softmax=True) - e) <= 3e-5 * (1 + e))


def test_convolution_runs_packed_pointwise_weight():
    # src/cpu/backend.rs:1490-1504
    w = np.array([1.0, 2.0, 3.0, 4.0], F32).reshape(2, 2, 1, 1)
    x = np.array([1.0, 2.0, 10.0, 20.0], F32).reshape(1, 2, 1, 2)
    out = oracle.conv2d(x, w, np.array([0.5, -0.5], F32))
    assert out.reshape(-1).tolist() == [21.5, 42.5, 42.5, 85.5]


def test_transposed_convolution_uses_io_weight_layout():
    # src/cpu/backend.rs:1849-1866
    w = np.ones((1, 1, 2, 2), F32)
    x = np.array([1.0, 2.0], F32).reshape(1, 1, 1, 2)
    out = oracle.conv_transpose2x2(x, w, np.array([0.5], F32))
    assert out.shape == (1, 1, 2, 4)
    assert out.reshape(-1).tolist() == [1.5, 1.5, 2.5, 2.5, 1.5, 1.5, 2.5, 2.5]


def test_transposed_convolution_matches_brute_force():
    # out[o, 2y+ky, 2x+kx] = sum_c in[c, y, x] W[c, o, ky, kx] + b[o] (src/cpu/ops.rs:1232-1267)
    rng = np.random.default_rng(0)
    x = rng.standard_normal((2, 3, 4, 5)).astype(F32)
    w = rng.standard_normal((3, 2, 2, 2)).astype(F32)
    b = rng.standard_normal(2).astype(F32)
    ref = np.zeros((2, 2, 8, 10))
    for ky in range(2):
        for kx in range(2):
            ref[:, :, ky::2, kx::2] = np.einsum("ncyx,co->noyx", x.astype(np.float64), w[:, :, ky, kx])
    ref += b[None, :, None, None]
    assert np.max(np.abs(oracle.conv_transpose2x2(x, w, b) - ref)) < 1e-5


def brute_conv(x, w, b, stride, pads, groups):
    n, c, h, wd = x.shape
    co, cg, kh, kw = w.shape
    ho = (h + pads[0] + pads[2] - kh) // stride[0] + 1
    wo = (wd + pads[1] + pads[3] - kw) // stride[1] + 1
    xp = np.zeros((n, c, h + pads[0] + pads[2], wd + pads[1] + pads[3]))
    xp[:, :, pads[0]:pads[0] + h, pads[1]:pads[1] + wd] = x
    out = np.zeros((n, co, ho, wo))
    opg = co // groups
    for o in range(co):
        g = o // opg
        for ky in range(kh):
            for kx in range(kw):
                patch = xp[:, g * cg:(g + 1) * cg, ky:ky + stride[0] * ho:stride[0], kx:kx + stride[1] * wo:stride[1]]
                out[:, o] += np.einsum("ncyx,c->nyx", patch, w[o, :, ky, kx])
    if b is not None:
        out += b[None, :, None, None]
    return out


@pytest.mark.parametrize("shape,wshape,stride,pads,groups", [
    ((1, 3, 9, 11), (8, 3, 3, 3), (2, 2), (1, 1, 1, 1), 1),      # stem 3x3 s2
    ((2, 4, 7, 6), (2, 4, 2, 2), (1, 1), (0, 0, 1, 1), 1),       # 2x2 pad bottom/right
    ((1, 6, 8, 9), (6, 1, 3, 3), (2, 2), (1, 1, 1, 1), 6),       # depthwise s2
    ((1, 4, 5, 12), (4, 1, 1, 7), (1, 1), (0, 3, 0, 3), 4),      # depthwise 1x7
    ((1, 5, 6, 7), (3, 5, 1, 1), (1, 1), (0, 0, 0, 0), 1),       # pointwise
    ((1, 4, 8, 10), (4, 4, 5, 5), (1, 1), (2, 2, 2, 2), 1),      # dense 5x5
    ((1, 6, 12, 10), (6, 1, 3, 3), (2, 1), (1, 1, 1, 1), 6),     # recognizer stride [2,1]
])
def test_convolution_matches_brute_force(shape, wshape, stride, pads, groups):
    # ops::conv (src/cpu/ops.rs:385-826), brute-force reference as
    # direct_spatial_six_row_blocks_match_scalar (src/cpu/backend.rs:1715-1805)
    rng = np.random.default_rng(sum(shape))
    x = rng.standard_normal(shape).astype(F32)
    w = rng.standard_normal(wshape).astype(F32)
    b = rng.standard_normal(wshape[0]).astype(F32)
    got = oracle.conv2d(x, w, b, stride, pads, groups, act="relu")
    ref = np.maximum(brute_conv(x.astype(np.float64), w.astype(np.float64), b, stride, pads, groups), 0)
    assert got.shape == ref.shape
    assert np.max(np.abs(got - ref)) < 5e-5 * (1 + np.max(np.abs(ref)))


def test_layer_norm_normalizes_the_last_dimension():
    # src/cpu/backend.rs:1474-1487
    w = np.ones(3, F32)
    b = np.zeros(3, F32)
    r0 = oracle.layer_norm([1.0, 2.0, 3.0], w, b, 1e-5)
    r1 = oracle.layer_norm([4.0, 4.0, 4.0], w, b, 1e-5)
    assert abs(float(np.sum(r0))) < 1e-5
    assert np.all(np.abs(r1) < 1e-6)


def test_layer_norm_closed_form():
    rng = np.random.default_rng(3)
    v = rng.standard_normal(120).astype(F32) * 3 + 1
    w = rng.standard_normal(120).astype(F32)
    b = rng.standard_normal(120).astype(F32)
    vd = v.astype(np.float64)
    ref = (vd - vd.mean()) / np.sqrt(vd.var() + 1e-6) * w + b
    assert np.max(np.abs(oracle.layer_norm(v, w, b, 1e-6) - ref)) < 2e-5


def test_softmax_is_normalized_and_ordered():
    # src/cpu/kernels/mod.rs:2999-3021
    x = np.array([-3.0, 0.5, 2.0, -0.25, 1.0, 0.0, -1.0], F32)
    e = np.exp(x.astype(np.float64) - x.max())
    e /= e.sum()
    got = oracle.softmax(x)
    assert abs(float(got.sum()) - 1.0) < 2e-6
    assert np.all(np.abs(got - e) < 2e-6)
    assert int(np.argmax(got)) == 2


def test_residual_mul_preserves_two_step_rounding():
    # src/cpu/kernels/mod.rs:3040-3053: fma(fma(v, g, 0), 1, v)
    for i in range(37):
        v = F32((i - 19.0) / 7.0)
        scaled = F32(np.float64(v) * np.float64(F32(0.375)))
        assert oracle.residual_mul(float(v), 0.375) == float(F32(np.float64(scaled) + np.float64(v)))
    # A case where one fused rounding differs from the two-step result.
    rng = np.random.default_rng(1)
    found = False
    for _ in range(20000):
        v, g = F32(rng.standard_normal()), F32(rng.standard_normal())
        two = F32(np.float64(F32(np.float64(v) * np.float64(g))) + np.float64(v))
        fused = F32(np.float64(v) * np.float64(g) + np.float64(v))
        if two != fused:
            assert oracle.residual_mul(float(v), float(g)) == float(two)
            found = True
            break
    assert found


def test_relu_and_max_pool_ignore_a_single_nan():
    # src/cpu/kernels/mod.rs:3055-3069
    assert oracle.act("relu", float("nan")) == 0.0
    x = np.ones((1, 1, 1, 17), F32)
    x[0, 0, 0, 0] = np.nan
    x[0, 0, 0, 1] = 2.0
    assert oracle.max_pool_same(x)[0, 0, 0, 0] == 2.0


def test_max_pool_same_upper_brute_force():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1, 2, 5, 6)).astype(F32)
    xp = np.full((1, 2, 6, 7), -np.inf, F32)
    xp[:, :, :5, :6] = x
    ref = np.maximum(np.maximum(xp[:, :, :5, :6], xp[:, :, 1:, :6]), np.maximum(xp[:, :, :5, 1:], xp[:, :, 1:, 1:]))
    assert np.array_equal(oracle.max_pool_same(x), ref)


def test_avg_pool_3x2():
    x = np.arange(2 * 3 * 6 * 8, dtype=F32).reshape(2, 3, 6, 8) * F32(0.37)
    got = oracle.avg_pool_3x2(x)
    ref = x.reshape(2, 3, 2, 3, 4, 2).astype(np.float64).mean(axis=(3, 5))
    assert got.shape == (2, 3, 2, 4)
    assert np.max(np.abs(got - ref)) < 1e-5


def test_fused_upsample_add_matches_resize_then_add():
    # src/cpu/model.rs:2141-2161
    upper = (np.arange(24, dtype=F32) - 9.0).reshape(2, 2, 2, 3) * F32(0.125)
    feature = (np.arange(96, dtype=F32) - 31.0).reshape(2, 2, 4, 6) * F32(0.0625)
    expected = feature + upper.repeat(2, axis=2).repeat(2, axis=3)
    assert np.array_equal(oracle.upsample_add(feature, upper, 2), expected)


def test_fused_upsample_cat_matches_reversed_neck_layout():
    # src/cpu/model.rs:2163-2194
    def make(shape, off):
        return (off + np.arange(np.prod(shape), dtype=F32) * F32(0.25)).reshape(shape)

    feats = [make((2, 1, 1, 2), 100.0), make((2, 2, 2, 4), 10.0), make((2, 1, 4, 8), -20.0)]
    scales = [4, 2, 1]
    expected = np.concatenate([f.repeat(s, 2).repeat(s, 3) for f, s in zip(feats, scales)], axis=1)
    got = oracle.upsample_cat(feats, scales)
    assert got.shape == (2, 4, 4, 8)
    assert np.array_equal(got, expected)


def test_rank_one_conv_matches_dense_fused_weight():
    # src/cpu/model.rs:2213-2268
    ci, co, k, h, w = 4, 5, 9, 11, 19
    sp = k * k
    dw = ((np.arange(ci * sp) * 17 % 43).astype(F32) - 21.0) / 97.0
    pw = ((np.arange(co * ci) * 11 % 29).astype(F32) - 14.0) / 31.0
    fused = (pw.reshape(co, ci, 1) * dw.reshape(1, ci, sp)).reshape(co, ci, k, k).astype(F32)
    bias = ((np.arange(co)).astype(F32) - 2.0) / 13.0
    x = ((np.arange(ci * h * w) * 23 % 61).astype(F32) - 30.0).reshape(1, ci, h, w) / F32(37.0)
    dense = oracle.conv2d(x, fused, bias, (1, 1), (4, 4, 4, 4), 1)
    dwf, pwf = oracle.factor_rank_one(fused)
    mid = oracle.conv2d(x, dwf, None, (1, 1), (4, 4, 4, 4), ci)
    rank1 = oracle.conv2d(mid, pwf, bias)
    assert np.max(np.abs(dense - rank1)) < 2e-5


def test_rank_one_factorization_rejects_nonseparable_weight():
    # src/cpu/model.rs:2270-2277
    w = np.zeros((2, 1, 3, 3), F32)
    w.reshape(-1)[0] = 1.0
    w.reshape(-1)[10] = 1.0
    with pytest.raises(RuntimeError, match="rank-one"):
        oracle.factor_rank_one(w)


def test_fuses_intraclass_weights_into_center_axes():
    # src/cpu/model.rs:2279-2328
    co, ci, k = 2, 2, 3
    sym = np.arange(co * ci * k * k, dtype=F32).reshape(co, ci, k, k)
    vert = (100 + np.arange(co * ci * k, dtype=F32)).reshape(co, ci, k, 1)
    hor = (200 + np.arange(co * ci * k, dtype=F32)).reshape(co, ci, 1, k)
    w, b = oracle.fuse_intraclass(sym, [1.0, 2.0], vert, [3.0, 4.0], hor, [5.0, 6.0])
    c = k // 2
    expected = sym.copy()
    expected[:, :, :, c] += vert[:, :, :, 0]
    expected[:, :, c, :] += hor[:, :, 0, :]
    assert np.array_equal(w, expected)
    assert b.tolist() == [9.0, 12.0]


def test_fused_intraclass_conv_matches_three_padded_branches():
    # src/cpu/model.rs:2330-2407
    co, ci, k = 2, 3, 5

    def pat(n, mul, scale):
        return ((np.arange(n) * mul % 31).astype(F32) - 15.0) * F32(scale)

    sw = pat(co * ci * k * k, 7, 0.01).reshape(co, ci, k, k)
    vw = pat(co * ci * k, 11, 0.015).reshape(co, ci, k, 1)
    hw = pat(co * ci * k, 13, 0.012).reshape(co, ci, 1, k)
    sb, vb, hb = np.array([0.07, -0.03], F32), np.array([-0.02, 0.05], F32), np.array([0.01, -0.04], F32)
    x = pat(ci * 7 * 8, 17, 0.02).reshape(1, ci, 7, 8)
    p = k // 2
    expected = (oracle.conv2d(x, sw, sb, (1, 1), (p, p, p, p)) + oracle.conv2d(x, vw, vb, (1, 1), (p, 0, p, 0))
                + oracle.conv2d(x, hw, hb, (1, 1), (0, p, 0, p)))
    fw, fb = oracle.fuse_intraclass(sw, sb, vw, vb, hw, hb)
    actual = oracle.conv2d(x, fw, fb, (1, 1), (p, p, p, p))
    assert np.all(np.abs(actual - expected) <= 2e-5 * np.maximum(np.abs(expected), 1.0))


def test_attention_context_matches_closed_form():
    # RecAttention::forward (src/cpu/model.rs:1703-1725) at the recognizer
    # shapes (40, 120, 8) / (40, 192, 8), as src/gpu/runtime.rs:3054-3107.
    rng = np.random.default_rng(2)
    for t, hidden, heads in ((3, 4, 2), (40, 120, 8), (40, 192, 8)):
        qkv = rng.standard_normal((2, t, 3 * hidden)).astype(F32)
        hd = hidden // heads
        q = qkv[:, :, :hidden].reshape(2, t, heads, hd).transpose(0, 2, 1, 3).astype(np.float64)
        kk = qkv[:, :, hidden:2 * hidden].reshape(2, t, heads, hd).transpose(0, 2, 1, 3).astype(np.float64)
        v = qkv[:, :, 2 * hidden:].reshape(2, t, heads, hd).transpose(0, 2, 1, 3).astype(np.float64)
        s = q @ kk.transpose(0, 1, 3, 2) * hd ** -0.5
        s = np.exp(s - s.max(-1, keepdims=True))
        s /= s.sum(-1, keepdims=True)
        ref = (s @ v).transpose(0, 2, 1, 3).reshape(2, t, hidden)
        assert np.max(np.abs(oracle.attention_context(qkv, heads) - ref)) < 5e-5


def from_fn(width, height, f):
    img = np.zeros((height, width, 3), np.uint8)
    for y in range(height):
        for x in range(width):
            img[y, x] = [v % 256 for v in f(x, y)]
    return img


def test_preprocess_matches_scalar_quad_bilinear_pipeline():
    # fused_parallel_preprocess_matches_the_scalar_pipeline (src/preprocess.rs:181-227)
    img = from_fn(37, 29, lambda x, y: (x * 7 + y * 3, x * 2 + y * 5, x * 3 + y * 7))
    corners = np.array([[2.25, 1.75], [34.5, 3.0], [32.75, 27.0], [1.0, 25.5]], F32)
    width, height = 41, 23
    mean, std = (0.485, 0.456, 0.406), (0.229, 0.224, 0.225)
    got = oracle.preprocess(img, corners, width, height, width, True)
    one = F32(1.0)
    for y in range(height):
        v = (F32(y) + F32(0.5)) / F32(height)
        for x in range(width):
            u = (F32(x) + F32(0.5)) / F32(width)
            top = corners[0] * (one - u) + corners[1] * u
            bottom = corners[3] * (one - u) + corners[2] * u
            pt = top * (one - v) + bottom * v
            sx = min(max(pt[0] - F32(0.5), F32(0)), F32(36))
            sy = min(max(pt[1] - F32(0.5), F32(0)), F32(28))
            x0, y0 = int(np.floor(sx)), int(np.floor(sy))
            x1, y1 = min(x0 + 1, 36), min(y0 + 1, 28)
            tx, ty = sx - F32(x0), sy - F32(y0)
            pix = []
            for c in range(3):
                t_ = F32(img[y0, x0, c]) * (one - tx) + F32(img[y0, x1, c]) * tx
                b_ = F32(img[y1, x0, c]) * (one - tx) + F32(img[y1, x1, c]) * tx
                pix.append(min(max(np.floor(t_ * (one - ty) + b_ * ty + F32(0.5)), 0), 255))
            bgr = [pix[2], pix[1], pix[0]]
            for c in range(3):
                expected = (bgr[c] / 255.0 - mean[c]) / std[c]
                assert abs(got[c, y, x] - expected) < 2e-6


def test_recognizer_preprocess_pads_and_tracks_content_width():
    # recognizer_pads_and_tracks_content_width (src/preprocess.rs:161-179):
    # an 80x20 crop scales to content width ceil(48*80/20) = 192 of 320.
    img = np.full((20, 80, 3), 127, np.uint8)
    corners = np.array([[0, 0], [80, 0], [80, 20], [0, 20]], F32)
    content = -(-48 * 80 // 20)
    assert content == 192
    got = oracle.preprocess(img, corners, 320, 48, content, False)
    assert got.shape == (3, 48, 320)
    assert abs(got[0, 0, 0] - (127 / 255 - 0.5) / 0.5) < 1e-6
    assert got[0, 0, content] == 0.0
    assert np.all(got[:, :, content:] == 0.0)


def test_identity_geometry_preprocess_equals_pixel_normalisation():
    # Identity corners land on pixel centres; rounding returns the pixel.
    import seeded

    rgb = seeded.seeded_rgb(32, 64, 9)
    got = oracle.preprocess(rgb, [[0, 0], [64, 0], [64, 32], [0, 32]], 64, 32, 64, True)
    assert np.array_equal(got, seeded.normalize_identity(rgb, True))


def test_bf16_emulation_rounds_and_resets():
    # The bf16 storage emulation moves the output by the size of bf16
    # rounding (not zero, far below the signal) and is off again afterwards.
    import seeded
    from helpers import model_path

    x = seeded.seeded_batch(1, 64, 96, 3)
    path = model_path("det", "tiny")
    ref = oracle.Model("det", path, "tiny").forward(x)
    oracle.set_bf16(True)
    try:
        emu = oracle.Model("det", path, "tiny").forward(x)
    finally:
        oracle.set_bf16(False)
    again = oracle.Model("det", path, "tiny").forward(x)
    d = np.abs(emu - ref)
    assert 1e-4 < d.max() < 0.2 and d.mean() < 2e-2
    assert np.array_equal(again, ref)
