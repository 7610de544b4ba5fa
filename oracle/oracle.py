"""ctypes wrapper of the CPU parity oracle (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg load
this module, as the checker or the CPU baseline.  The oracle restates the
reference CPU path; see oracle.cpp for the per-function citations.
"""

from __future__ import annotations

import ctypes
import os
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

SIZE_CODE = {"medium": 0, "small": 1, "tiny": 2}
ACT = {"none": 0, "relu": 1, "gelu": 2, "silu": 3, "hsig6": 4, "hsig5": 5, "hswish": 6, "sigmoid": 7}

_lib = None
_F = ctypes.POINTER(ctypes.c_float)
_I = ctypes.POINTER(ctypes.c_int)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle library not built: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(str(LIB_PATH))
        L.oracle_last_error.restype = ctypes.c_char_p
        L.oracle_detector_load.restype = ctypes.c_void_p
        L.oracle_detector_load.argtypes = [ctypes.c_char_p, ctypes.c_int]
        L.oracle_recognizer_load.restype = ctypes.c_void_p
        L.oracle_recognizer_load.argtypes = [ctypes.c_char_p, ctypes.c_int]
        L.oracle_model_free.argtypes = [ctypes.c_void_p]
        L.oracle_forward.argtypes = [ctypes.c_void_p, _F, _I, _F, ctypes.c_size_t, _I]
        L.oracle_erf.restype = ctypes.c_float
        L.oracle_erf.argtypes = [ctypes.c_float]
        L.oracle_act.restype = ctypes.c_float
        L.oracle_act.argtypes = [ctypes.c_int, ctypes.c_float]
        L.oracle_residual_mul.restype = ctypes.c_float
        L.oracle_residual_mul.argtypes = [ctypes.c_float, ctypes.c_float]
        L.oracle_layer_norm.argtypes = [_F, _F, _F, ctypes.c_int, ctypes.c_float]
        L.oracle_softmax.argtypes = [_F, ctypes.c_int]
        L.oracle_linear.argtypes = [_F, ctypes.c_long, ctypes.c_int, _F, ctypes.c_int, _F, ctypes.c_int,
                                    ctypes.c_int, _F]
        L.oracle_set_threads.argtypes = [ctypes.c_int]
        _lib = L
    return _lib


def _f(a):
    return a.ctypes.data_as(_F)


def _i(a):
    return a.ctypes.data_as(_I)


def _check(rc):
    if rc != 0:
        raise RuntimeError(lib().oracle_last_error().decode())


def set_threads(n):
    lib().oracle_set_threads(int(n))


class Model:
    """A loaded oracle detector or recognizer."""

    def __init__(self, kind, path, size):
        L = lib()
        load = L.oracle_detector_load if kind == "det" else L.oracle_recognizer_load
        self.handle = load(str(path).encode(), SIZE_CODE[size])
        if not self.handle:
            raise RuntimeError(L.oracle_last_error().decode())
        self.kind = kind
        self.size = size

    def output_len(self, shape):
        n, _, h, w = shape
        if self.kind == "det":
            return n * h * w
        classes = 6906 if self.size == "tiny" else 18710
        return n * (w // 4 // 2 + 1) * classes

    def forward(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        shape = np.array(x.shape, dtype=np.int32)
        cap = self.output_len(x.shape)
        out = np.empty(cap, dtype=np.float32)
        oshape = np.zeros(4, dtype=np.int32)
        _check(lib().oracle_forward(ctypes.c_void_p(self.handle), _f(x), _i(shape), _f(out), cap, _i(oshape)))
        dims = [int(d) for d in oshape if d > 0]
        return out[: int(np.prod(dims))].reshape(dims)

    def __del__(self):
        if getattr(self, "handle", None):
            lib().oracle_model_free(ctypes.c_void_p(self.handle))
            self.handle = None


def preprocess(rgb, corners, canvas_w, canvas_h, content_w, detector=True):
    rgb = np.ascontiguousarray(rgb, dtype=np.uint8)
    sh, sw = rgb.shape[:2]
    c = np.ascontiguousarray(np.asarray(corners, dtype=np.float32).reshape(8))
    out = np.empty((3, canvas_h, canvas_w), dtype=np.float32)
    _check(lib().oracle_preprocess(rgb.ctypes.data_as(ctypes.c_void_p), sw, sh, _f(c), canvas_w, canvas_h,
                                   content_w, int(detector), _f(out)))
    return out


def conv2d(x, w, bias=None, stride=(1, 1), pads=(0, 0, 0, 0), groups=1, act="none"):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, c, h, wd = x.shape
    co, _, kh, kw = w.shape
    ho = (h + pads[0] + pads[2] - kh) // stride[0] + 1
    wo = (wd + pads[1] + pads[3] - kw) // stride[1] + 1
    out = np.empty((n, co, ho, wo), dtype=np.float32)
    oshape = np.zeros(4, dtype=np.int32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    _check(lib().oracle_conv2d(_f(x), _i(np.array(x.shape, np.int32)), _f(w), _i(np.array(w.shape, np.int32)),
                               None if b is None else _f(b), int(stride[0]), int(stride[1]),
                               _i(np.array(pads, np.int32)), int(groups), ACT[act], _f(out), _i(oshape)))
    return out


def conv_transpose2x2(x, w, bias=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, c, h, wd = x.shape
    out = np.empty((n, w.shape[1], 2 * h, 2 * wd), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    _check(lib().oracle_conv_transpose2x2(_f(x), _i(np.array(x.shape, np.int32)), _f(w),
                                          _i(np.array(w.shape, np.int32)), None if b is None else _f(b), _f(out)))
    return out


def linear(x, w, bias=None, act="none", softmax=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    k = w.shape[1]
    rows = x.size // k
    out = np.empty(x.shape[:-1] + (w.shape[0],), dtype=np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    _check(lib().oracle_linear(_f(x), rows, k, _f(w), w.shape[0], None if b is None else _f(b), ACT[act],
                               int(softmax), _f(out)))
    return out


def softmax(v):
    v = np.array(v, dtype=np.float32)
    lib().oracle_softmax(_f(v), v.size)
    return v


def layer_norm(v, w, b, eps):
    v = np.array(v, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    lib().oracle_layer_norm(_f(v), _f(w), _f(b), v.size, ctypes.c_float(eps))
    return v


def erf(x):
    return lib().oracle_erf(float(x))


def act(name, x):
    return lib().oracle_act(ACT[name], float(x))


def residual_mul(v, g):
    return lib().oracle_residual_mul(float(v), float(g))


def max_pool_same(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    _check(lib().oracle_max_pool_same(_f(x), _i(np.array(x.shape, np.int32)), _f(out)))
    return out


def avg_pool_3x2(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n, c, h, w = x.shape
    out = np.empty((n, c, (h - 3) // 3 + 1, (w - 2) // 2 + 1), dtype=np.float32)
    oshape = np.zeros(4, dtype=np.int32)
    _check(lib().oracle_avg_pool_3x2(_f(x), _i(np.array(x.shape, np.int32)), _f(out), _i(oshape)))
    return out


def upsample_add(feature, upper, scale):
    f = np.array(feature, dtype=np.float32)
    u = np.ascontiguousarray(upper, dtype=np.float32)
    _check(lib().oracle_upsample_add(_f(f), _i(np.array(f.shape, np.int32)), _f(u),
                                     _i(np.array(u.shape, np.int32)), int(scale)))
    return f


def upsample_cat(features, scales):
    feats = [np.ascontiguousarray(f, dtype=np.float32) for f in features]
    ptrs = (ctypes.POINTER(ctypes.c_float) * len(feats))(*[_f(f) for f in feats])
    shapes = np.array([f.shape for f in feats], dtype=np.int32).reshape(-1)
    n, _, h, w = feats[0].shape
    c = sum(f.shape[1] for f in feats)
    out = np.empty((n, c, h * scales[0], w * scales[0]), dtype=np.float32)
    oshape = np.zeros(4, dtype=np.int32)
    _check(lib().oracle_upsample_cat(len(feats), ptrs, _i(shapes), _i(np.array(scales, np.int32)), _f(out),
                                     _i(oshape)))
    return out


def attention_context(qkv, heads):
    qkv = np.ascontiguousarray(qkv, dtype=np.float32)
    b, t, h3 = qkv.shape
    out = np.empty((b, t, h3 // 3), dtype=np.float32)
    _check(lib().oracle_attention(_f(qkv), b, t, h3 // 3, heads, _f(out)))
    return out


def factor_rank_one(w):
    w = np.ascontiguousarray(w, dtype=np.float32)
    co, ci, k, _ = w.shape
    dw = np.empty((ci, 1, k, k), dtype=np.float32)
    pw = np.empty((co, ci, 1, 1), dtype=np.float32)
    _check(lib().oracle_factor_rank_one(_f(w), ci, co, k, _f(dw), _f(pw)))
    return dw, pw


def fuse_intraclass(sym, sb, vert, vb, hor, hb):
    sym = np.array(sym, dtype=np.float32)
    sb = np.array(sb, dtype=np.float32)
    co, ci, k, _ = sym.shape
    _check(lib().oracle_fuse_intraclass(_f(sym), _f(sb), _f(np.ascontiguousarray(vert, np.float32)),
                                        _f(np.ascontiguousarray(vb, np.float32)),
                                        _f(np.ascontiguousarray(hor, np.float32)),
                                        _f(np.ascontiguousarray(hb, np.float32)), co, ci, k))
    return sym, sb


# ------------------------------------------------------------ greedy CTC
PROBABILITY_EPSILON = np.float32(1e-8)  # src/ocr.rs:23


def _argmax_last(row):
    """``argmax`` (src/ocr.rs:1171-1177): ``max_by(total_cmp)`` keeps the last
    of equal maxima.  Rows are finite (checked by the caller), so the only
    place ``total_cmp`` differs from ``>=`` is -0.0 against +0.0, which a
    probability row cannot hold as its maximum."""
    return int(row.shape[0] - 1 - np.argmax(row[::-1]))


def _row_probability(row, value):
    """``row_probability`` (src/ocr.rs:1158-1169): the value itself when the
    row is already a distribution (all >= 0, sum within 0.01 of 1), else its
    max-subtracted softmax probability.  The sum is taken in float32
    (pairwise rather than sequential: a difference of order 1e-6 against the
    0.01 test)."""
    total = float(np.sum(row, dtype=np.float32))
    if np.all(row >= 0) and abs(total - 1.0) <= 0.01:
        return float(np.clip(np.float32(value), 0.0, 1.0))
    m = np.float32(np.max(row))
    den = np.sum(np.exp((row - m).astype(np.float32)), dtype=np.float32)
    return float(np.clip(np.float32(np.exp(np.float32(value - m)) / den), 0.0, 1.0))


def ctc_greedy_decode(values, dictionary_len, content_width, input_width):
    """``decode_ctc_greedy_for_input`` (src/ocr.rs:800-853) on one item's
    [T, V] rows.  Returns (emitted class indices, score); the caller maps
    class c to dictionary[c - 1], or to a space for the implicit last class
    when V == len(dictionary) + 2."""
    values = np.asarray(values, dtype=np.float32)
    t, classes = values.shape
    if classes != dictionary_len + 1 and classes != dictionary_len + 2:
        raise ValueError("class count does not match the dictionary")
    if content_width == 0 or content_width > input_width:
        raise ValueError("content width outside 1..=input width")
    if not np.all(np.isfinite(values)):
        raise ValueError("non-finite recognizer output")
    valid = min(max(-(-content_width * t // input_width), 1), t)
    tokens, log_score, previous = [], 0.0, 0
    for step in range(valid):
        row = values[step]
        cls = _argmax_last(row)
        if cls != 0 and cls != previous:
            tokens.append(cls)
            p = max(np.float32(_row_probability(row, row[cls])), PROBABILITY_EPSILON)
            log_score += float(np.log(np.float64(p)))
        previous = cls
    score = float(np.float32(np.exp(log_score / len(tokens)))) if tokens else 0.0
    return tokens, score


# ------------------------------------------------------------ DB postprocess
DB_DEFAULTS = dict(binary_threshold=0.2, box_threshold=0.4, min_area=3, unclip_ratio=1.4, max_boxes=1000)


def extract_detections(values, transform, binary_threshold=0.2, box_threshold=0.4, min_area=3, unclip_ratio=1.4,
                       max_boxes=1000):
    """``extract_detections`` (src/ocr.rs:723-790) on one [H, W] probability map.

    ``transform`` = (source_width, source_height, content_width,
    content_height) of ``DetectorTransform`` (src/ocr.rs:32-74).  Returns
    (polygons [n, 4, 2], scores [n], anisotropy [n]); anisotropy is a
    diagnostic of how well the component's principal axis is determined.
    """
    v = np.ascontiguousarray(values, dtype=np.float32)
    h, w = v.shape
    tr = (ctypes.c_uint32 * 4)(*[int(t) for t in transform])
    count = ctypes.c_size_t()
    L = lib()
    fn = L.oracle_extract_detections
    fn.argtypes = [_F, ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_uint32), ctypes.c_float, ctypes.c_float,
                   ctypes.c_size_t, ctypes.c_float, ctypes.c_size_t, _F, ctypes.c_size_t,
                   ctypes.POINTER(ctypes.c_size_t)]
    args = (v.ctypes.data_as(_F), h, w, tr, binary_threshold, box_threshold, min_area, unclip_ratio, max_boxes)
    if fn(*args, None, 0, ctypes.byref(count)) != 0:
        raise ValueError("invalid postprocess arguments or non-finite map")
    out = np.zeros((max(count.value, 1), 10), dtype=np.float32)
    fn(*args, out.ctypes.data_as(_F), out.shape[0], ctypes.byref(count))
    out = out[:count.value]
    return out[:, :8].reshape(-1, 4, 2), out[:, 8].copy(), out[:, 9].copy()


# ------------------------------------------------------------ test hooks
def fault_count():
    """Number of plantable wiring mistakes (fault ids 1 .. count-1; 0 = none)."""
    L = lib()
    L.oracle_fault_count.restype = ctypes.c_int
    return int(L.oracle_fault_count())


def set_fault(fault):
    """Plants wiring mistake ``fault`` (0 = none) in models loaded and run
    afterwards; see ``enum Fault`` in oracle.cpp.  Tests only."""
    L = lib()
    L.oracle_set_fault.argtypes = [ctypes.c_int]
    L.oracle_set_fault(int(fault))


def set_tracing(on):
    """Records named intermediate tensors of the next forward passes."""
    L = lib()
    L.oracle_set_tracing.argtypes = [ctypes.c_int]
    L.oracle_set_tracing(int(bool(on)))


def traced(name):
    """The traced tensor ``name`` of the last forward pass (KeyError if absent)."""
    L = lib()
    fn = L.oracle_trace_get
    fn.restype = ctypes.c_long
    fn.argtypes = [ctypes.c_char_p, _F, ctypes.c_size_t, _I]
    shape = np.zeros(4, dtype=np.int32)
    n = fn(name.encode(), None, 0, _i(shape))
    if n == 0:
        raise KeyError(name)
    out = np.empty(n, dtype=np.float32)
    fn(name.encode(), _f(out), n, _i(shape))
    return out.reshape([int(d) for d in shape if d > 0])


def set_bf16(on):
    """bf16 storage emulation for models run afterwards: the tensors a bf16
    plan stores, and its matrix-core weights, rounded to bf16 (tests only)."""
    L = lib()
    L.oracle_set_bf16.argtypes = [ctypes.c_int]
    L.oracle_set_bf16(int(bool(on)))


def bf16_log():
    """The rounding points of the last forward run with the bf16 emulation
    on, in order: "A <value>" (an activation value rounded to bf16) and
    "W <layer>" (a layer's weights rounded to bf16)."""
    L = lib()
    fn = L.oracle_bf16_log
    fn.argtypes = [ctypes.c_char_p, ctypes.c_size_t]
    fn.restype = ctypes.c_long
    n = fn(None, 0)
    buf = ctypes.create_string_buffer(n)
    fn(buf, n)
    return buf.value.decode().splitlines()


def round_bf16(values):
    """The emulation's float32 -> bf16 rounding (nearest even; NaN kept),
    elementwise, as float32."""
    L = lib()
    fn = L.oracle_round_bf16
    fn.argtypes = [_F, _F, ctypes.c_size_t]
    fn.restype = None
    x = np.ascontiguousarray(values, dtype=np.float32)
    out = np.empty_like(x)
    fn(_f(x), _f(out), x.size)
    return out


def set_reverse_sums(on):
    """Accumulate matrix products, depthwise convs and attention sums last
    term first, for models run afterwards (tests only)."""
    L = lib()
    L.oracle_set_reverse_sums.argtypes = [ctypes.c_int]
    L.oracle_set_reverse_sums(int(bool(on)))
