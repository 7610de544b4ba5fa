"""Python mirror of the reference's ``ppocr_rs::gpu`` API over the C ABI.

The classes follow the reference's direct-model API (``src/gpu/mod.rs:3-13``):
``Gpu`` (``Gpu::new``, ``upload_rgb``), ``Detector`` / ``Recognizer``
(``load``, ``forward``, ``forward_image``, ``benchmark``) returning
``ModelOutput`` (shape + values), and ``GpuError`` carrying the status code
of the reference ``gpu::Error`` variant (``src/gpu/error.rs:9-45``).

Everything runs in ``libppocr_hip.so`` (include/ppocr_hip.h); this module
only marshals arguments.  It raises when the library is missing: there is no
fallback path.
"""

from __future__ import annotations

import ctypes
import os
import pathlib
from dataclasses import dataclass

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = pathlib.Path(os.environ.get("PPOCR_HIP_LIB", HERE / "libppocr_hip.so"))

SIZE_CODE = {"medium": 0, "small": 1, "tiny": 2}
PRECISION = {"f32": 0, "bf16": 1}
STATUS = {
    0: "Ok", 1: "ReadFile", 2: "Safetensors", 3: "TensorNotFound", 4: "UnsupportedDtype",
    5: "ShapeMismatch", 6: "TensorSizeOverflow", 7: "TensorByteLength", 8: "InvalidTensorRange",
    9: "InvalidModel", 10: "InvalidInput", 11: "Gpu",
}

# Every symbol include/ppocr_hip.h declares.
EXPORTS = (
    "ppocr_hip_last_error", "ppocr_hip_create", "ppocr_hip_destroy", "ppocr_hip_device_info", "ppocr_hip_detector_load",
    "ppocr_hip_recognizer_load", "ppocr_hip_model_free", "ppocr_hip_output_shape", "ppocr_hip_forward",
    "ppocr_hip_upload_rgb", "ppocr_hip_image_free", "ppocr_hip_forward_image", "ppocr_hip_preprocess",
    "ppocr_hip_benchmark", "ppocr_hip_benchmark_stream", "ppocr_hip_profile", "ppocr_hip_memory_report",
    "ppocr_hip_recognizer_load_greedy", "ppocr_detector_input_plan", "ppocr_recognizer_batch_width",
    "ppocr_recognition_input_plan", "ppocr_ctc_greedy_decode", "ppocr_db_default_options",
    "ppocr_hip_db_postprocess", "ppocr_hip_db_postprocess_static", "ppocr_hip_detect", "ppocr_hip_detect_image", "ppocr_engine_default_options",
    "ppocr_hip_engine_load", "ppocr_hip_engine_free", "ppocr_hip_engine_recognize", "ppocr_ocr_result_lines",
    "ppocr_ocr_result_tokens", "ppocr_ocr_result_sizes", "ppocr_ocr_result_free",
)


class GpuError(RuntimeError):
    """A failed C-ABI call; ``kind`` names the reference ``gpu::Error`` variant."""

    def __init__(self, code, message):
        super().__init__(f"{STATUS.get(code, code)}: {message}")
        self.code = code
        self.kind = STATUS.get(code, str(code))


class DbOptions(ctypes.Structure):
    """``DetectorPostprocessOptions`` (src/ocr.rs:231-269)."""

    _fields_ = [("binary_threshold", ctypes.c_float), ("box_threshold", ctypes.c_float),
                ("min_area", ctypes.c_size_t), ("unclip_ratio", ctypes.c_float), ("max_boxes", ctypes.c_size_t)]


class DetectorTransform(ctypes.Structure):
    """``DetectorTransform`` (src/ocr.rs:32-74)."""

    _fields_ = [("source_width", ctypes.c_uint32), ("source_height", ctypes.c_uint32),
                ("content_width", ctypes.c_uint32), ("content_height", ctypes.c_uint32)]


class GpuInfoStruct(ctypes.Structure):
    """``ppocr_gpu_info``: ``GpuInfo`` (src/gpu/runtime.rs:17-21) plus HIP device facts."""

    _fields_ = [("name", ctypes.c_char * 256), ("backend", ctypes.c_char * 16), ("arch", ctypes.c_char * 64),
                ("device", ctypes.c_int), ("integrated", ctypes.c_int), ("compute_units", ctypes.c_int),
                ("wavefront_size", ctypes.c_int), ("total_memory", ctypes.c_size_t)]


@dataclass
class GpuInfo:
    """``GpuInfo`` (src/gpu/runtime.rs:17-21): name, backend, device type, and
    the HIP architecture, compute units, wavefront size and memory."""

    name: str
    backend: str
    device_type: str
    arch: str
    device: int
    compute_units: int
    wavefront_size: int
    total_memory: int


class _Detection(ctypes.Structure):
    _fields_ = [("polygon", ctypes.c_float * 8), ("score", ctypes.c_float)]


@dataclass
class Detection:
    """``Detection`` (src/ocr.rs:225-229): corners [4, 2] in source pixels, score."""

    polygon: np.ndarray
    score: float


def db_options(**kw):
    o = DbOptions(0.2, 0.4, 3, 1.4, 1000)
    for k, v in kw.items():
        setattr(o, k, v)
    return o


def _transforms(transforms):
    ts = [tuple(int(v) for v in t) for t in transforms]
    return (DetectorTransform * len(ts))(*[DetectorTransform(*t) for t in ts]), len(ts)


def _collect(call, n, max_boxes):
    """Runs a postprocess entry point with room for max_boxes detections per
    image (the most it can return); one list of Detection per image."""
    counts = (ctypes.c_size_t * n)()
    total = ctypes.c_size_t()
    buf = (_Detection * (n * max_boxes))()
    _check(call(buf, n * max_boxes, counts, ctypes.byref(total)))
    rows = np.frombuffer(buf, dtype=np.float32).reshape(n * max_boxes, 9)[:total.value].copy()
    polygons = rows[:, :8].reshape(-1, 4, 2)
    scores = rows[:, 8].tolist()
    out, k = [], 0
    for i in range(n):
        c = counts[i]
        out.append([Detection(polygons[j], scores[j]) for j in range(k, k + c)])
        k += c
    return out


class KernelStat(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 64), ("kernel", ctypes.c_char * 32), ("avg_ms", ctypes.c_double),
                ("flops", ctypes.c_double), ("bytes", ctypes.c_double), ("bound", ctypes.c_int)]


_lib = None
_SZ = ctypes.POINTER(ctypes.c_size_t)
_F = ctypes.POINTER(ctypes.c_float)
_D = ctypes.POINTER(ctypes.c_double)
_VP = ctypes.c_void_p


def lib():
    """Loads libppocr_hip.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"HIP backend library missing: {LIB_PATH} (build it with make -C ppocr-rs_amd)")
        L = ctypes.CDLL(str(LIB_PATH))
        L.ppocr_hip_last_error.restype = ctypes.c_char_p
        L.ppocr_hip_create.argtypes = [ctypes.c_int, ctypes.POINTER(_VP)]
        L.ppocr_hip_destroy.argtypes = [_VP]
        L.ppocr_hip_device_info.argtypes = [_VP, _VP]
        L.ppocr_hip_detector_load.argtypes = [_VP, ctypes.c_char_p, ctypes.c_int, _SZ, ctypes.c_int,
                                              ctypes.POINTER(_VP)]
        L.ppocr_hip_recognizer_load.argtypes = [_VP, ctypes.c_char_p, ctypes.c_int, _SZ, ctypes.c_int, _VP,
                                                ctypes.POINTER(_VP)]
        L.ppocr_hip_model_free.argtypes = [_VP]
        L.ppocr_hip_output_shape.argtypes = [_VP, _SZ, _SZ]
        L.ppocr_hip_forward.argtypes = [_VP, _F, ctypes.c_size_t, _F, ctypes.c_size_t]
        L.ppocr_hip_upload_rgb.argtypes = [_VP, ctypes.c_uint32, ctypes.c_uint32, _VP, ctypes.c_size_t,
                                           ctypes.POINTER(_VP)]
        L.ppocr_hip_image_free.argtypes = [_VP]
        L.ppocr_hip_forward_image.argtypes = [_VP, _VP, _F, _SZ, ctypes.c_size_t, _F, ctypes.c_size_t]
        L.ppocr_hip_preprocess.argtypes = [_VP, _VP, _F, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                           ctypes.c_int, _F]
        L.ppocr_hip_benchmark.argtypes = [_VP, _F, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, _D]
        L.ppocr_hip_benchmark_stream.argtypes = [_VP, _F, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, _D]
        L.ppocr_hip_profile.argtypes = [_VP, _F, ctypes.c_size_t, ctypes.c_size_t, ctypes.POINTER(KernelStat),
                                        ctypes.c_size_t, _SZ]
        L.ppocr_hip_memory_report.argtypes = [_VP, _SZ, _SZ, _SZ]
        L.ppocr_hip_recognizer_load_greedy.argtypes = L.ppocr_hip_recognizer_load.argtypes
        _U32 = ctypes.POINTER(ctypes.c_uint32)
        L.ppocr_detector_input_plan.argtypes = [ctypes.c_uint32, ctypes.c_uint32, _U32, _U32, _U32]
        L.ppocr_recognizer_batch_width.argtypes = [_F, ctypes.c_size_t, _SZ]
        L.ppocr_recognition_input_plan.argtypes = [_F, ctypes.c_size_t, _SZ]
        L.ppocr_ctc_greedy_decode.argtypes = [_F, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t,
                                              ctypes.c_size_t, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int32),
                                              _SZ, _F]
        _T = ctypes.POINTER(DetectorTransform)
        _O = ctypes.POINTER(DbOptions)
        _D8 = ctypes.POINTER(_Detection)
        L.ppocr_db_default_options.argtypes = [_O]
        L.ppocr_db_default_options.restype = None
        L.ppocr_hip_db_postprocess.argtypes = [_VP, _F, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_size_t, _T, _O,
                                               _D8, ctypes.c_size_t, _SZ, _SZ]
        L.ppocr_hip_db_postprocess_static.argtypes = L.ppocr_hip_db_postprocess.argtypes
        L.ppocr_hip_detect.argtypes = [_VP, _F, ctypes.c_size_t, _T, _O, _D8, ctypes.c_size_t, _SZ, _SZ]
        L.ppocr_hip_detect_image.argtypes = [_VP, _VP, _F, ctypes.c_size_t, _T, _O, _D8, ctypes.c_size_t, _SZ,
                                             _SZ]
        _lib = L
    return _lib


def _check(code):
    if code != 0:
        raise GpuError(code, lib().ppocr_hip_last_error().decode(errors="replace"))


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(_F)


def _sizes(values):
    arr = (ctypes.c_size_t * len(values))(*[int(v) for v in values])
    return arr


@dataclass
class ModelOutput:
    """``gpu::ModelOutput`` (src/gpu/model.rs:37-41)."""

    shape: list
    values: np.ndarray

    def array(self):
        return self.values.reshape(self.shape)


class Gpu:
    """``gpu::Gpu`` (src/gpu/runtime.rs:94-229): one device, stream and arena."""

    def __init__(self, device=0):
        h = _VP()
        _check(lib().ppocr_hip_create(int(device), ctypes.byref(h)))
        self.handle = h
        self._children = []

    def info(self):
        """``Gpu::info`` (src/gpu/runtime.rs:169-171)."""
        s = GpuInfoStruct()
        _check(lib().ppocr_hip_device_info(self.handle, ctypes.byref(s)))
        return GpuInfo(s.name.decode(errors="replace"), s.backend.decode(), "IntegratedGpu" if s.integrated else
                       "DiscreteGpu", s.arch.decode(errors="replace"), s.device, s.compute_units, s.wavefront_size,
                       s.total_memory)

    def upload_rgb(self, rgb):
        """``Gpu::upload_rgb``: RGB8 HWC array -> device image."""
        rgb = np.ascontiguousarray(rgb, dtype=np.uint8)
        if rgb.ndim != 3 or rgb.shape[2] != 3:
            raise ValueError("expected an HxWx3 uint8 image")
        h = _VP()
        _check(lib().ppocr_hip_upload_rgb(self.handle, rgb.shape[1], rgb.shape[0], rgb.ctypes.data_as(_VP), rgb.size,
                                          ctypes.byref(h)))
        return GpuImage(self, h, rgb.shape[1], rgb.shape[0])

    def preprocess(self, image, corners, canvas_w, canvas_h, content_width=None, detector=True):
        """Device ``prepare_detector`` / ``prepare_recognizer`` of one quad -> [3, h, w]."""
        c, cp = _f32(np.asarray(corners, dtype=np.float32).reshape(8))
        out = np.empty((3, canvas_h, canvas_w), dtype=np.float32)
        _check(lib().ppocr_hip_preprocess(self.handle, image.handle, cp, canvas_w, canvas_h,
                                          canvas_w if content_width is None else content_width, int(detector),
                                          out.ctypes.data_as(_F)))
        return out

    def db_postprocess(self, prob, transforms, **options):
        """``extract_detections`` (src/ocr.rs:723-790) on the device for host
        maps [N, H, W] (or [H, W]); one list of Detection per map."""
        p = np.ascontiguousarray(prob, dtype=np.float32)
        if p.ndim == 2:
            p = p[None]
        n, h, w = p.shape
        tr, nt = _transforms(transforms)
        if nt != n:
            raise ValueError("one transform per map")
        o = db_options(**options)
        return _collect(lambda buf, cap, counts, total: lib().ppocr_hip_db_postprocess(
            self.handle, p.ctypes.data_as(_F), n, h, w, tr, ctypes.byref(o), buf, cap, counts, total), n, o.max_boxes)

    def db_postprocess_static(self, prob, transforms, **options):
        """As ``db_postprocess``, through the entry point that allocates no
        device memory (maps and work arrays in the library's static scratch)."""
        p = np.ascontiguousarray(prob, dtype=np.float32)
        if p.ndim == 2:
            p = p[None]
        n, h, w = p.shape
        tr, nt = _transforms(transforms)
        if nt != n:
            raise ValueError("one transform per map")
        o = db_options(**options)
        return _collect(lambda buf, cap, counts, total: lib().ppocr_hip_db_postprocess_static(
            self.handle, p.ctypes.data_as(_F), n, h, w, tr, ctypes.byref(o), buf, cap, counts, total), n, o.max_boxes)

    def close(self):
        for child in self._children:
            child.close()
        self._children.clear()
        if self.handle:
            lib().ppocr_hip_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class GpuImage:
    def __init__(self, gpu, handle, width, height):
        self.gpu, self.handle, self.width, self.height = gpu, handle, width, height

    def close(self):
        if self.handle:
            lib().ppocr_hip_image_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _Model:
    def __init__(self, gpu, handle, input_shape):
        self.gpu = gpu
        self.handle = handle
        self.input_shape = tuple(int(v) for v in input_shape)
        shape = (ctypes.c_size_t * 4)()
        rank = ctypes.c_size_t()
        _check(lib().ppocr_hip_output_shape(handle, shape, ctypes.byref(rank)))
        self.output_shape = [int(shape[i]) for i in range(rank.value)]
        self.output_len = int(np.prod(self.output_shape))
        gpu._children.append(self)

    def forward(self, nchw):
        """``forward(&[f32]) -> ModelOutput`` (src/gpu/model.rs:95-114, :222-237)."""
        x, xp = _f32(nchw)
        out = np.empty(self.output_len, dtype=np.float32)
        _check(lib().ppocr_hip_forward(self.handle, xp, x.size, out.ctypes.data_as(_F), out.size))
        return ModelOutput(list(self.output_shape), out)

    def forward_image(self, image, corners, content_widths=None):
        """``forward_image`` with per-item quads [N, 4, 2] and content widths [N]."""
        c, cp = _f32(np.asarray(corners, dtype=np.float32).reshape(-1, 8))
        n = c.shape[0]
        widths = None if content_widths is None else _sizes(content_widths)
        out = np.empty(self.output_len, dtype=np.float32)
        _check(lib().ppocr_hip_forward_image(self.handle, image.handle, cp, widths, n, out.ctypes.data_as(_F),
                                             out.size))
        return ModelOutput(list(self.output_shape), out)

    def benchmark(self, nchw, warmup=5, runs=30):
        """Per-run milliseconds, device-only like ``benchmark_nchw`` (src/gpu/runtime.rs:1798-1830)."""
        x, xp = _f32(nchw)
        samples = (ctypes.c_double * runs)()
        _check(lib().ppocr_hip_benchmark(self.handle, xp, x.size, warmup, runs, samples))
        return list(samples)

    def benchmark_stream(self, nchw, warmup, runs):
        """Total milliseconds of ``runs`` back-to-back passes (inputs resident in HBM)."""
        x, xp = _f32(nchw)
        total = ctypes.c_double()
        _check(lib().ppocr_hip_benchmark_stream(self.handle, xp, x.size, warmup, runs, ctypes.byref(total)))
        return total.value

    def profile(self, nchw, runs=10):
        x, xp = _f32(nchw)
        count = ctypes.c_size_t()
        _check(lib().ppocr_hip_profile(self.handle, xp, x.size, 1, None, 0, ctypes.byref(count)))
        stats = (KernelStat * count.value)()
        _check(lib().ppocr_hip_profile(self.handle, xp, x.size, runs, stats, count.value, ctypes.byref(count)))
        return [dict(name=s.name.decode(), kernel=s.kernel.decode(), avg_ms=s.avg_ms, flops=s.flops, bytes=s.bytes,
                     bound={1: "mfma", 2: "valu"}.get(s.bound, "hbm")) for s in stats]

    def memory_report(self):
        a, u, w = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
        _check(lib().ppocr_hip_memory_report(self.handle, ctypes.byref(a), ctypes.byref(u), ctypes.byref(w)))
        return {"arena_bytes": a.value, "unplanned_bytes": u.value, "weight_bytes": w.value}

    def close(self):
        if self.handle:
            lib().ppocr_hip_model_free(self.handle)
            self.handle = None


class Detector(_Model):
    """``gpu::Detector`` (src/gpu/model.rs:44-148)."""

    @classmethod
    def load(cls, gpu, path, size, input_shape, precision="f32"):
        h = _VP()
        _check(lib().ppocr_hip_detector_load(gpu.handle, str(path).encode(), SIZE_CODE[size], _sizes(input_shape),
                                             PRECISION[precision], ctypes.byref(h)))
        return cls(gpu, h, input_shape)

    def detect(self, nchw, transforms, **options):
        """Forward + device DB postprocess; one list of Detection per image."""
        x, xp = _f32(nchw)
        tr, n = _transforms(transforms)
        o = db_options(**options)
        return _collect(lambda buf, cap, counts, total: lib().ppocr_hip_detect(
            self.handle, xp, x.size, tr, ctypes.byref(o), buf, cap, counts, total), n, o.max_boxes)

    def detect_image(self, image, corners, transforms, **options):
        """``forward_image`` + device DB postprocess (quads [N, 4, 2])."""
        c, cp = _f32(np.asarray(corners, dtype=np.float32).reshape(-1, 8))
        tr, n = _transforms(transforms)
        o = db_options(**options)
        return _collect(lambda buf, cap, counts, total: lib().ppocr_hip_detect_image(
            self.handle, image.handle, cp, c.shape[0], tr, ctypes.byref(o), buf, cap, counts, total), n,
            o.max_boxes)


class Recognizer(_Model):
    """``gpu::Recognizer`` (src/gpu/model.rs:150-266)."""

    @classmethod
    def load(cls, gpu, path, size, input_shape, precision="f32", share_weights=None, greedy=False):
        """``Recognizer::load`` / ``load_with_shared_weights``.  With ``greedy``
        the classifier is fused with per-step greedy CTC decoding and the
        output is [N, T, 2] (class index, probability) per time step."""
        h = _VP()
        entry = lib().ppocr_hip_recognizer_load_greedy if greedy else lib().ppocr_hip_recognizer_load
        _check(entry(gpu.handle, str(path).encode(), SIZE_CODE[size], _sizes(input_shape), PRECISION[precision],
                     share_weights.handle if share_weights is not None else None, ctypes.byref(h)))
        return cls(gpu, h, input_shape)


# ------------------------------------------------------------ host geometry

def detector_input_plan(width, height, max_side=736):
    """``DetectorInputPlan::new`` (src/ocr.rs:86-101): (input_width, input_height)
    for an image; ``max_side=None`` applies ``default_detector_ratio``."""
    w, h = ctypes.c_uint32(), ctypes.c_uint32()
    ms = None if max_side is None else ctypes.byref(ctypes.c_uint32(int(max_side)))
    _check(lib().ppocr_detector_input_plan(int(width), int(height), ms, ctypes.byref(w), ctypes.byref(h)))
    return w.value, h.value


def recognizer_batch_width(polygons):
    """``recognizer_batch_width`` (src/ocr.rs:206-219) over quads [n, 4, 2]."""
    c, cp = _f32(np.asarray(polygons, dtype=np.float32).reshape(-1, 8))
    out = ctypes.c_size_t()
    _check(lib().ppocr_recognizer_batch_width(cp, c.shape[0], ctypes.byref(out)))
    return out.value


def recognition_input_plan(polygon, input_width):
    """``recognition_input_plan`` (src/ocr.rs:154-171): the crop's content width."""
    c, cp = _f32(np.asarray(polygon, dtype=np.float32).reshape(8))
    out = ctypes.c_size_t()
    _check(lib().ppocr_recognition_input_plan(cp, int(input_width), ctypes.byref(out)))
    return out.value


@dataclass
class DecodedText:
    """``DecodedText`` (src/ocr.rs:268-272)."""

    text: str
    score: float


def ctc_greedy_decode(steps, dictionary, classes, content_width, input_width):
    """``decode_ctc_greedy_for_input`` (src/ocr.rs:800-853) for one item of a
    greedy recognizer's output ([T, 2]: class index, probability)."""
    s, sp = _f32(np.asarray(steps, dtype=np.float32).reshape(-1, 2))
    t = s.shape[0]
    tokens = (ctypes.c_int32 * max(t, 1))()
    n = ctypes.c_size_t()
    score = ctypes.c_float()
    _check(lib().ppocr_ctc_greedy_decode(sp, t, int(classes), len(dictionary), int(content_width), int(input_width),
                                         tokens, ctypes.byref(n), ctypes.byref(score)))
    space = classes == len(dictionary) + 2
    text = "".join(" " if space and tokens[i] == classes - 1 else dictionary[tokens[i] - 1] for i in range(n.value))
    return DecodedText(text, score.value)


# ------------------------------------------------------------ OCR engine

class EngineOptions(ctypes.Structure):
    """``OcrOptions`` (src/ocr.rs:285-299) for this backend."""

    _fields_ = [("detector_size", ctypes.c_int), ("recognizer_size", ctypes.c_int), ("precision", ctypes.c_int),
                ("postprocess", DbOptions), ("detector_max_side", ctypes.c_uint32), ("greedy", ctypes.c_int)]


class _OcrLine(ctypes.Structure):
    _fields_ = [("polygon", ctypes.c_float * 8), ("detection_score", ctypes.c_float),
                ("recognition_score", ctypes.c_float), ("token_offset", ctypes.c_size_t),
                ("token_count", ctypes.c_size_t)]


@dataclass
class OcrLine:
    """``OcrLine`` (src/ocr.rs:330-341)."""

    polygon: np.ndarray
    detection_score: float
    text: str
    recognition_score: float
    tokens: list


@dataclass
class OcrResult:
    """``OcrResult`` (src/ocr.rs:343-368)."""

    source_size: tuple
    detector_input_size: tuple
    lines: list

    def text(self):
        return "\n".join(line.text for line in self.lines if line.text)


def _engine_lib():
    L = lib()
    if not getattr(L, "_engine_ready", False):
        L.ppocr_engine_default_options.argtypes = [ctypes.POINTER(EngineOptions)]
        L.ppocr_engine_default_options.restype = None
        L.ppocr_hip_engine_load.argtypes = [_VP, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t,
                                            ctypes.POINTER(EngineOptions), ctypes.POINTER(_VP)]
        L.ppocr_hip_engine_free.argtypes = [_VP]
        L.ppocr_hip_engine_recognize.argtypes = [_VP, _VP, ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(_VP)]
        L.ppocr_ocr_result_lines.argtypes = [_VP, _SZ]
        L.ppocr_ocr_result_lines.restype = ctypes.POINTER(_OcrLine)
        L.ppocr_ocr_result_tokens.argtypes = [_VP, _SZ]
        L.ppocr_ocr_result_tokens.restype = ctypes.POINTER(ctypes.c_int32)
        L.ppocr_ocr_result_sizes.argtypes = [_VP, ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_uint32)]
        L.ppocr_ocr_result_sizes.restype = None
        L.ppocr_ocr_result_free.argtypes = [_VP]
        L._engine_ready = True
    return L


class OcrEngine:
    """``OcrEngine`` (src/ocr.rs:354-600) running on this backend."""

    def __init__(self, gpu, handle, dictionary, classes):
        self.gpu, self.handle, self.dictionary, self.classes = gpu, handle, list(dictionary), classes
        gpu._children.append(self)

    @classmethod
    def load(cls, gpu, detector_model, recognizer_model, dictionary, detector_size="tiny", recognizer_size="tiny",
             precision="f32", detector_max_side=736, greedy=True, **postprocess):
        """``OcrEngine::load`` (src/ocr.rs:416-494); ``dictionary`` is the list of
        entries (``load_dictionary``, src/ocr.rs:792-798)."""
        L = _engine_lib()
        o = EngineOptions()
        L.ppocr_engine_default_options(ctypes.byref(o))
        o.detector_size, o.recognizer_size = SIZE_CODE[detector_size], SIZE_CODE[recognizer_size]
        o.precision = PRECISION[precision]
        o.detector_max_side = 0 if detector_max_side is None else int(detector_max_side)
        o.greedy = int(bool(greedy))
        for k, v in postprocess.items():
            setattr(o.postprocess, k, v)
        h = _VP()
        _check(L.ppocr_hip_engine_load(gpu.handle, str(detector_model).encode(), str(recognizer_model).encode(),
                                       len(dictionary), ctypes.byref(o), ctypes.byref(h)))
        return cls(gpu, h, dictionary, 6906 if recognizer_size == "tiny" else 18710)

    def recognize(self, rgb):
        """``OcrEngine::recognize`` (src/ocr.rs:497-522) on an HxWx3 uint8 image."""
        L = _engine_lib()
        rgb = np.ascontiguousarray(rgb, dtype=np.uint8)
        if rgb.ndim != 3 or rgb.shape[2] != 3:
            raise ValueError("expected an HxWx3 uint8 image")
        r = _VP()
        _check(L.ppocr_hip_engine_recognize(self.handle, rgb.ctypes.data_as(_VP), rgb.shape[1], rgb.shape[0],
                                            ctypes.byref(r)))
        try:
            n, nt = ctypes.c_size_t(), ctypes.c_size_t()
            lines = L.ppocr_ocr_result_lines(r, ctypes.byref(n))
            toks = L.ppocr_ocr_result_tokens(r, ctypes.byref(nt))
            src, det = (ctypes.c_uint32 * 2)(), (ctypes.c_uint32 * 2)()
            L.ppocr_ocr_result_sizes(r, src, det)
            space = self.classes == len(self.dictionary) + 2
            out = []
            for i in range(n.value):
                ln = lines[i]
                ids = [int(toks[ln.token_offset + k]) for k in range(ln.token_count)]
                text = "".join(" " if space and c == self.classes - 1 else self.dictionary[c - 1] for c in ids)
                out.append(OcrLine(np.array(ln.polygon[:], np.float32).reshape(4, 2), float(ln.detection_score),
                                   text, float(ln.recognition_score), ids))
            return OcrResult((src[0], src[1]), (det[0], det[1]), out)
        finally:
            L.ppocr_ocr_result_free(r)

    def close(self):
        if self.handle:
            _engine_lib().ppocr_hip_engine_free(self.handle)
            self.handle = None
