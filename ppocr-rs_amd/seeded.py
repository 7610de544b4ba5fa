"""Seeded PP-OCRv6 weights and inputs at the exact tensor names and shapes.

The pinned Hugging Face checkpoints cannot be fetched offline, so every model
is exercised with seeded weights that carry the reference's tensor names and
shapes.  The schema below restates the loaders of the reference CPU path:

* LCNet backbone, blocks and stems: ``src/cpu/model.rs:409-809``
  (``ConvBnAct``, ``SqueezeExcitation``, ``LcNetBlock``, ``LargeStem``,
  ``SmallStem``) and the stage tables ``:1648-1673`` / ``:2057-2122``.
* RepLK FPN neck (tiny/small): ``src/cpu/model.rs:1069-1254``.
* Medium neck with rank-one 9x9 convs and intraclass blocks:
  ``src/cpu/model.rs:811-1067``.
* DB head: ``src/cpu/model.rs:1419-1521``.
* Recognizer heads: ``src/cpu/model.rs:1675-1936``.

Tensor counts equal the loader checks in ``src/gpu/model.rs:11-16``
(271/271/350 detectors, 150/250/269 recognizers); parameter totals equal the
pinned file sizes in ``models.json`` less the safetensors header.

Generator rules (seeded, every tensor F32):

* conv/linear weights ``N(0,1) * gain / sqrt(fan_in)``; biases ``N(0, 0.02)``;
* BatchNorm ``weight = 1 + N(0,0.02)``, ``bias = N(0,0.02)``,
  ``running_mean = N(0,0.02)``, ``running_var = 1 + |N(0,0.02)|`` so that the
  fold ``gamma / sqrt(var + 1e-5)`` is finite (``src/cpu/model.rs:397``);
* LayerNorm ``weight = 1 + N(0,0.02)``, ``bias = N(0,0.02)``;
* the medium detector's 9x9 projection/lateral weights are outer products
  ``pw[o,c] * dw[c,ky,kx]`` so the reference loader's rank-one factorisation
  accepts them (``src/cpu/model.rs:221-369``).
"""

from __future__ import annotations

import numpy as np

SIZES = ("tiny", "small", "medium")
SIZE_CODE = {"medium": 0, "small": 1, "tiny": 2}

DETECTOR_TENSORS = {"medium": 350, "small": 271, "tiny": 271}
RECOGNIZER_TENSORS = {"medium": 269, "small": 250, "tiny": 150}
RECOGNIZER_CLASSES = {"medium": 18710, "small": 18710, "tiny": 6906}

# (kind, name, shape, fan_in)
#   kind: w (conv/linear weight), b (bias), bnw/bnb/bnm/bnv (batch norm),
#         lnw/lnb (layer norm), r1 (rank-one 9x9 weight)


class _Schema:
    def __init__(self):
        self.items = []

    def add(self, kind, name, shape, fan_in=0):
        self.items.append((kind, name, tuple(int(s) for s in shape), int(fan_in)))

    def conv(self, prefix, ci, co, kernel, groups=1, bias=False):
        kh, kw = kernel
        self.add("w", f"{prefix}.weight", (co, ci // groups, kh, kw), ci // groups * kh * kw)
        if bias:
            self.add("b", f"{prefix}.bias", (co,))

    def bn(self, prefix, channels):
        for kind, leaf in (("bnw", "weight"), ("bnb", "bias"), ("bnm", "running_mean"),
                           ("bnv", "running_var")):
            self.add(kind, f"{prefix}.{leaf}", (channels,))

    def conv_bn(self, prefix, ci, co, kernel, groups=1, bias=False, norm="normalization"):
        self.conv(f"{prefix}.convolution", ci, co, kernel, groups, bias)
        self.bn(f"{prefix}.{norm}", co)

    def linear(self, prefix, fin, fout):
        self.add("w", f"{prefix}.weight", (fout, fin), fin)
        self.add("b", f"{prefix}.bias", (fout,))

    def layer_norm(self, prefix, features):
        self.add("lnw", f"{prefix}.weight", (features,))
        self.add("lnb", f"{prefix}.bias", (features,))


def detector_stages(channels):
    """``detector_stages_for_channels`` (src/cpu/model.rs:1648-1673)."""
    s1, s2, s3, s4 = channels
    return [
        [(s1, s1, (1, 1), True), (s1, s1, (1, 1), False)],
        [(s1, s2, (2, 2), False), (s2, s2, (1, 1), True), (s2, s2, (1, 1), False)],
        [(s2, s3, (2, 2), False), (s3, s3, (1, 1), True), (s3, s3, (1, 1), False),
         (s3, s3, (1, 1), True), (s3, s3, (1, 1), False)],
        [(s3, s4, (2, 2), False), (s4, s4, (1, 1), True), (s4, s4, (1, 1), False)],
    ]


def recognizer_stages(size):
    """``recognizer_stages``/``small_``/``tiny_`` (src/cpu/model.rs:2057-2122)."""
    if size == "medium":
        return [
            [(128, 128, (1, 1), True)],
            [(128, 256, (1, 1), False), (256, 256, (1, 1), False), (256, 256, (1, 1), True)],
            [(256, 512, (2, 1), False)] + [(512, 512, (1, 1), i % 2 == 0) for i in range(6)],
            [(512, 768, (2, 1), False), (768, 768, (1, 1), True), (768, 768, (1, 1), False)],
        ]
    if size == "small":
        return [
            [(96, 96, (1, 1), True)],
            [(96, 96, (1, 1), False), (96, 96, (1, 1), False)],
            [(96, 192, (2, 1), False)] + [(192, 192, (1, 1), i % 2 == 0) for i in range(6)],
            [(192, 384, (2, 1), False), (384, 384, (1, 1), True), (384, 384, (1, 1), False)],
        ]
    return [
        [(48, 48, (1, 1), True)],
        [(48, 48, (1, 1), False)],
        [(48, 96, (2, 1), False), (96, 96, (1, 1), True), (96, 96, (1, 1), False)],
        [(96, 160, (2, 1), False), (160, 160, (1, 1), True), (160, 160, (1, 1), False),
         (160, 160, (1, 1), False)],
    ]


DETECTOR_CHANNELS = {"medium": (128, 256, 512, 896), "small": (48, 96, 192, 384),
                     "tiny": (32, 48, 64, 160)}
DETECTOR_STEM = {"medium": (64, 128), "small": (24, 48), "tiny": (16, 32)}
DETECTOR_NECK = {"medium": 256, "small": 96, "tiny": 64}
FPN_KERNEL = {"small": 7, "tiny": 5}
RECOGNIZER_STEM = {"medium": (64, 128), "small": (48, 96), "tiny": (24, 48)}
SVTR = {"medium": (768, 192, 768), "small": (384, 120, 240)}  # input, hidden, mlp


def _backbone(s, stem, stages, small_stem=False):
    enc = "model.backbone.encoder"
    mid, out = stem
    if small_stem:
        s.conv_bn(f"{enc}.convolution.conv1", 3, mid, (3, 3))
        s.conv_bn(f"{enc}.convolution.conv2", mid, out, (3, 3))
    else:
        s.conv_bn(f"{enc}.convolution.stem1", 3, mid, (3, 3))
        s.conv_bn(f"{enc}.convolution.stem2a", mid, mid // 2, (2, 2))
        s.conv_bn(f"{enc}.convolution.stem2b", mid // 2, mid, (2, 2))
        s.conv_bn(f"{enc}.convolution.stem3", mid * 2, mid, (3, 3))
        s.conv_bn(f"{enc}.convolution.stem4", mid, out, (1, 1))
    for si, stage in enumerate(stages):
        for bi, (ci, co, stride, se) in enumerate(stage):
            p = f"{enc}.blocks.{si}.blocks.{bi}"
            residual = ci == co and tuple(stride) == (1, 1)
            if residual:
                s.conv(f"{p}.token_conv", ci, ci, (3, 3), groups=ci, bias=True)
            else:
                s.conv_bn(f"{p}.token_conv", ci, ci, (3, 3), groups=ci)
            if se:
                s.conv(f"{p}.token_squeeze_excitation.convolutions.0", ci, ci // 4, (1, 1), bias=True)
                s.conv(f"{p}.token_squeeze_excitation.convolutions.2", ci // 4, ci, (1, 1), bias=True)
            s.conv_bn(f"{p}.channel_conv1", ci, ci * 2, (1, 1))
            s.conv_bn(f"{p}.channel_conv2", ci * 2, co, (1, 1))


def detector_schema(size):
    s = _Schema()
    chans = DETECTOR_CHANNELS[size]
    _backbone(s, DETECTOR_STEM[size], detector_stages(chans))
    nc = DETECTOR_NECK[size]
    if size == "medium":
        neck = "model.neck"
        for i, c in enumerate(chans):
            s.conv(f"{neck}.input_channel_adjustment_convolution.{i}", c, 256, (1, 1))
        for i in range(4):
            s.add("r1", f"{neck}.input_feature_projection_convolution.{i}.weight", (64, 256, 9, 9), 256 * 81)
            s.add("b", f"{neck}.input_feature_projection_convolution.{i}.bias", (64,))
        for i in range(3):
            s.conv(f"{neck}.path_aggregation_head_convolution.{i}", 64, 64, (3, 3))
        for i in range(4):
            s.add("r1", f"{neck}.path_aggregation_lateral_convolution.{i}.weight", (64, 64, 9, 9), 64 * 81)
            s.add("b", f"{neck}.path_aggregation_lateral_convolution.{i}.bias", (64,))
        for i in range(4):
            p = f"{neck}.intraclass_blocks.{i}"
            s.conv(f"{p}.conv_reduce_channel", 64, 32, (1, 1), bias=True)
            for ratio, k in (("longratio", 7), ("midratio", 5), ("shortratio", 3)):
                s.conv(f"{p}.symmetric_conv_long_{ratio}", 32, 32, (k, k), bias=True)
                s.conv(f"{p}.vertical_long_to_small_conv_{ratio}", 32, 32, (k, 1), bias=True)
                s.conv(f"{p}.horizontal_small_to_long_conv_{ratio}", 32, 32, (1, k), bias=True)
            s.conv_bn(f"{p}.conv_final", 32, 64, (1, 1), bias=True, norm="norm")
    else:
        k = FPN_KERNEL[size]
        for i, c in enumerate(chans):
            p = f"model.neck.insert_conv.{i}"
            s.conv(f"{p}.in_conv", c, nc, (1, 1))
            s.conv(f"{p}.squeeze_excitation_block.conv1", nc, nc // 4, (1, 1), bias=True)
            s.conv(f"{p}.squeeze_excitation_block.conv2", nc // 4, nc, (1, 1), bias=True)
        for i in range(4):
            p = f"model.neck.input_conv.{i}"
            s.conv(f"{p}.depthwise_convolution", nc, nc, (k, k), groups=nc, bias=True)
            s.conv(f"{p}.pointwise_convolution", nc, nc // 4, (1, 1))
            s.conv(f"{p}.squeeze_excitation_module.conv1", nc // 4, nc // 16, (1, 1), bias=True)
            s.conv(f"{p}.squeeze_excitation_module.conv2", nc // 16, nc // 4, (1, 1), bias=True)
    h = nc // 4
    s.conv_bn("head.conv_down", nc, h, (3, 3), norm="norm")
    s.add("w", "head.conv_up.convolution.weight", (h, h, 2, 2), h * 4)
    s.add("b", "head.conv_up.convolution.bias", (h,))
    s.bn("head.conv_up.norm", h)
    s.add("w", "head.conv_final.weight", (h, 1, 2, 2), h * 4)
    s.add("b", "head.conv_final.bias", (1,))
    return s.items


def recognizer_schema(size):
    s = _Schema()
    _backbone(s, RECOGNIZER_STEM[size], recognizer_stages(size), small_stem=(size == "tiny"))
    if size == "tiny":
        s.add("w", "head.conv1.weight", (160, 1, 5), 5)
        s.bn("head.norm1", 160)
        s.add("w", "head.conv2.weight", (160, 160, 1), 160)
        s.bn("head.norm2", 160)
        s.linear("head.fc1", 160, 80)
        s.linear("head.fc2", 80, RECOGNIZER_CLASSES[size])
    else:
        ci, h, mlp = SVTR[size]
        e = "head.encoder"
        s.conv_bn(f"{e}.conv_block.0", ci, h, (1, 1))
        s.conv_bn(f"{e}.conv_block.1", ci, h, (1, 1))
        s.conv_bn(f"{e}.conv_block.2", h, h, (1, 7), groups=h)
        for i in range(2):
            p = f"{e}.svtr_block.{i}"
            s.layer_norm(f"{p}.layer_norm1", h)
            s.linear(f"{p}.self_attn.qkv", h, 3 * h)
            s.linear(f"{p}.self_attn.projection", h, h)
            s.layer_norm(f"{p}.layer_norm2", h)
            s.linear(f"{p}.mlp.fc1", h, mlp)
            s.linear(f"{p}.mlp.fc2", mlp, h)
        s.layer_norm(f"{e}.norm", h)
        s.linear("head.head", h, RECOGNIZER_CLASSES[size])
    return s.items


def schema(kind, size):
    return detector_schema(size) if kind == "det" else recognizer_schema(size)


def seeded_weights(kind, size, seed=0, gain=1.0, head_gain=None):
    """Returns ``{name: float32 array}`` for one model at the reference shapes."""
    rng = np.random.Generator(np.random.PCG64(seed))
    out = {}
    for k, name, shape, fan_in in schema(kind, size):
        n = int(np.prod(shape))
        if k == "w":
            g = gain
            if head_gain is not None and (name.startswith("head.head") or name.startswith("head.fc2")):
                g = head_gain
            v = rng.standard_normal(n) * (g / np.sqrt(fan_in))
        elif k == "r1":
            co, ci, kh, kw = shape
            pw = rng.standard_normal((co, ci)) * (gain / np.sqrt(ci))
            dw = rng.standard_normal((ci, kh * kw)) / np.sqrt(kh * kw)
            v = (pw.astype(np.float32)[:, :, None] * dw.astype(np.float32)[None, :, :]).reshape(-1)
        elif k in ("b", "bnb", "bnm", "lnb"):
            v = rng.standard_normal(n) * 0.02
        elif k in ("bnw", "lnw"):
            v = 1.0 + rng.standard_normal(n) * 0.02
        elif k == "bnv":
            v = 1.0 + np.abs(rng.standard_normal(n) * 0.02)
        else:
            raise ValueError(k)
        out[name] = np.ascontiguousarray(np.asarray(v, dtype=np.float32).reshape(shape))
    return out


# Per-model gains keep the seeded networks away from both collapse (a flat
# probability map / uniform softmax) and saturation (probabilities stuck at
# 0 or 1), so parity checks compare informative outputs.  They also keep the
# networks well conditioned: a 1e-7 relative perturbation of the input moves
# every output by at most ~1e-4 (tests/test_seeded_models.py), so the 1e-3
# parity tolerance measures kernel error rather than the amplification of
# fp32 rounding noise by an exploding network.
DEFAULT_GAINS = {
    ("det", "tiny"): (1.2, None), ("det", "small"): (1.16, None), ("det", "medium"): (1.12, None),
    ("rec", "tiny"): (1.3, 4.0), ("rec", "small"): (1.22, 1.0), ("rec", "medium"): (1.3, 0.5),
}


def write_weights(path, kind, size, seed=0, **kw):
    from safetensors.numpy import save_file

    if not kw:
        gain, head_gain = DEFAULT_GAINS[(kind, size)]
        kw = {"gain": gain, "head_gain": head_gain}
    save_file(seeded_weights(kind, size, seed, **kw), str(path))
    return path


def seeded_rgb(height, width, seed, pattern="uniform"):
    """Seeded RGB8 image (HWC).

    ``uniform``: every channel uniform in [0, 255].  ``blocks``: a light noise
    background (200-255) with random dark axis-aligned rectangles (0-60) until
    5-30 % of the pixels are covered, a text-like pattern.
    """
    rng = np.random.Generator(np.random.PCG64(seed))
    if pattern == "uniform":
        return rng.integers(0, 256, size=(height, width, 3), dtype=np.uint8)
    img = rng.integers(200, 256, size=(height, width, 3), dtype=np.uint8)
    mask = np.zeros((height, width), dtype=bool)
    target = rng.uniform(0.05, 0.30)
    while mask.mean() < target:
        rh = int(rng.integers(max(4, height // 64), max(5, height // 10)))
        rw = int(rng.integers(max(8, width // 40), max(9, width // 4)))
        y = int(rng.integers(0, max(1, height - rh)))
        x = int(rng.integers(0, max(1, width - rw)))
        mask[y:y + rh, x:x + rw] = True
        img[y:y + rh, x:x + rw] = rng.integers(0, 61, size=(rh, rw, 3), dtype=np.uint8)
    return img


DET_MEAN = (0.485, 0.456, 0.406)
DET_STD = (0.229, 0.224, 0.225)
REC_MEAN = (0.5, 0.5, 0.5)
REC_STD = (0.5, 0.5, 0.5)


def normalize_identity(rgb, detector=True):
    """BGR-normalised NCHW planes of an RGB8 image sampled at identity geometry.

    With corners equal to the full image and a canvas of the image's own size
    the reference's quad-bilinear sampler lands on pixel centres and rounds
    back to the pixel value (``src/preprocess/kernels.rs:94-165``), so the
    result is ``v * (1/(255 std)) + (-mean/std)`` per BGR channel, computed
    in float32 without fused multiply-add, as ``normalize`` does (``:167-170``).
    """
    mean, std = (DET_MEAN, DET_STD) if detector else (REC_MEAN, REC_STD)
    bgr = rgb[..., ::-1].astype(np.float32)
    out = np.empty((3,) + rgb.shape[:2], dtype=np.float32)
    for c in range(3):
        scale = np.float32(1.0) / (np.float32(255.0) * np.float32(std[c]))
        bias = np.float32(-np.float32(mean[c])) / np.float32(std[c])
        out[c] = bgr[..., c] * scale + bias
    return out


def seeded_batch(n, height, width, seed, detector=True, pattern="uniform"):
    """``[n, 3, height, width]`` float32 of ``n`` independent seeded images."""
    return np.stack([normalize_identity(seeded_rgb(height, width, seed + i, pattern), detector)
                     for i in range(n)])
