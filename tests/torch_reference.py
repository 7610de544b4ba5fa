"""Independent float64 PyTorch functional model of the PP-OCRv6 networks.

Test infrastructure only.  This is a second, separately written statement of
the reference CPU models (``src/cpu/model.rs``), used to pin the network
composition of the oracle (``oracle/oracle.cpp``): which tensor each residual
adds, the gate constants, the concat orders, the BN fold axes, the encoder's
skip/LayerNorm order.  It shares no code with the oracle and avoids its
load-time rewrites so that a misreading in one is unlikely to be repeated in
the other:

* batch norm runs as ``F.batch_norm`` on the unfolded statistics instead of
  being folded into the weights (``fold_batch_norm``, ``src/cpu/model.rs:371-407``;
  ``fold_transpose_batch_norm``, ``:1440-1477``);
* the medium neck's rank-one 9x9 convolutions run dense on the stored
  ``[O, I, 9, 9]`` weight instead of as depthwise + pointwise factors
  (``RankOneConv2d``, ``:165-219``);
* the intraclass blocks run their three branches (k x k, k x 1, 1 x k) and add
  them, instead of the fused kernel (``fuse_intraclass_conv``, ``:819-888``);
* every primitive is a library routine: ``F.conv2d``, ``F.conv_transpose2d``,
  ``F.max_pool2d``, ``F.avg_pool2d``, ``F.layer_norm``, ``torch.softmax``,
  ``F.gelu`` (exact erf), ``F.hardswish``, ``F.silu``.

Arithmetic is float64, so against the float32 oracle the difference is the
oracle's own rounding.  Module order and names follow the reference line by
line; each function cites the lines it restates.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

DTYPE = torch.float64

# Named intermediate tensors of the running forward pass, under the names the
# oracle's trace uses; a dict while ``forward(..., trace=...)`` runs.
_TRACE = None


def _t(name, value):
    if _TRACE is not None:
        _TRACE[name] = value.numpy().copy()
    return value


class Weights:
    """Safetensors tensors as float64 torch tensors, looked up by dotted name."""

    def __init__(self, tensors):
        self.t = {k: torch.from_numpy(np.asarray(v, dtype=np.float64)) for k, v in tensors.items()}

    @classmethod
    def load(cls, path):
        from safetensors.numpy import load_file

        return cls(load_file(str(path)))

    def __call__(self, name, shape=None):
        v = self.t[name]
        if shape is not None:
            assert tuple(v.shape) == tuple(shape), (name, tuple(v.shape), shape)
        return v


# ---------------------------------------------------------------- primitives
def pad_conv(x, w, bias=None, stride=(1, 1), pads=(0, 0, 0, 0), groups=1):
    """Conv with the reference's [top, left, bottom, right] pads (``src/cpu/ops.rs:419-434``)."""
    t, l, b, r = pads
    x = F.pad(x, (l, r, t, b))
    return F.conv2d(x, w, bias, stride=stride, groups=groups)


def batch_norm(x, wt, prefix):
    """Inference batch norm with eps 1e-5 (``src/cpu/model.rs:397``)."""
    return F.batch_norm(x, wt(f"{prefix}.running_mean"), wt(f"{prefix}.running_var"), wt(f"{prefix}.weight"),
                        wt(f"{prefix}.bias"), training=False, eps=1e-5)


def hard_sigmoid(x, alpha):
    """``into_hard_sigmoid(alpha, 0.5)`` (``src/cpu/model.rs:77-78``)."""
    return torch.clamp(x * alpha + 0.5, 0.0, 1.0)


def activation(x, name):
    if name == "none":
        return x
    if name == "relu":
        return F.relu(x)
    if name == "silu":
        return F.silu(x)
    if name == "gelu":
        return F.gelu(x)
    raise ValueError(name)


def conv(wt, prefix, x, stride=(1, 1), pads=(0, 0, 0, 0), groups=1, bias=False):
    """``Conv2d::load`` + forward (``src/cpu/model.rs:89-107``)."""
    return pad_conv(x, wt(f"{prefix}.weight"), wt(f"{prefix}.bias") if bias else None, stride, pads, groups)


def conv_bn_act(wt, prefix, x, stride=(1, 1), pads=(0, 0, 0, 0), groups=1, bias=False, norm="normalization",
                act="none"):
    """``ConvBnAct`` (``src/cpu/model.rs:409-454``): conv, batch norm, activation."""
    y = conv(wt, f"{prefix}.convolution", x, stride, pads, groups, bias)
    return activation(batch_norm(y, wt, f"{prefix}.{norm}"), act)


def nearest_up(x, scale):
    """Integer-scale nearest upsample, source ``floor(dst / scale)``
    (``upsample_add_nchw`` / ``upsample_and_cat_nchw``, ``src/cpu/model.rs:1265-1417``)."""
    return x if scale == 1 else x.repeat_interleave(scale, dim=2).repeat_interleave(scale, dim=3)


# ---------------------------------------------------------------- backbone
def squeeze_excitation(wt, prefix, x):
    """``SqueezeExcitation::forward`` (``src/cpu/model.rs:487-492``): x * hsig(1/6)."""
    pooled = x.mean(dim=(2, 3), keepdim=True)
    r = F.relu(conv(wt, f"{prefix}.convolutions.0", pooled, bias=True))
    g = hard_sigmoid(conv(wt, f"{prefix}.convolutions.2", r, bias=True), 1.0 / 6.0)
    return x * g


def lcnet_block(wt, prefix, x, ci, co, stride):
    """``LcNetBlock::forward`` (``src/cpu/model.rs:592-602``) with the pair's
    residual (``src/cpu/backend.rs:470-477``): the residual adds the tensor
    entering channel_conv1, i.e. after the token conv and the SE."""
    residual = ci == co and tuple(stride) == (1, 1)
    if residual:
        t = conv(wt, f"{prefix}.token_conv", x, stride, (1, 1, 1, 1), groups=ci, bias=True)
    else:
        t = conv_bn_act(wt, f"{prefix}.token_conv", x, stride, (1, 1, 1, 1), groups=ci)
    if f"{prefix}.token_squeeze_excitation.convolutions.0.weight" in wt.t:
        t = squeeze_excitation(wt, f"{prefix}.token_squeeze_excitation", t)
    h = conv_bn_act(wt, f"{prefix}.channel_conv1", t, act="gelu")
    o = conv_bn_act(wt, f"{prefix}.channel_conv2", h)
    return t + o if residual else o


def large_stem(wt, x):
    """``LargeStem::forward`` (``src/cpu/model.rs:684-692``), ReLU everywhere."""
    p = "model.backbone.encoder.convolution"
    e = conv_bn_act(wt, f"{p}.stem1", x, (2, 2), (1, 1, 1, 1), act="relu")
    br = conv_bn_act(wt, f"{p}.stem2a", e, pads=(0, 0, 1, 1), act="relu")
    br = conv_bn_act(wt, f"{p}.stem2b", br, pads=(0, 0, 1, 1), act="relu")
    pooled = F.max_pool2d(F.pad(e, (0, 1, 0, 1), value=float("-inf")), 2, 1)
    merged = torch.cat([pooled, br], dim=1)
    return conv_bn_act(wt, f"{p}.stem4", conv_bn_act(wt, f"{p}.stem3", merged, (2, 2), (1, 1, 1, 1), act="relu"),
                       act="relu")


def small_stem(wt, x):
    """``SmallStem::forward`` (``src/cpu/model.rs:730-732``): conv1+BN, GELU, conv2+BN."""
    p = "model.backbone.encoder.convolution"
    h = conv_bn_act(wt, f"{p}.conv1", x, (2, 2), (1, 1, 1, 1), act="gelu")
    return conv_bn_act(wt, f"{p}.conv2", h, (2, 2), (1, 1, 1, 1))


def detector_stage_specs(c1, c2, c3, c4):
    """``detector_stages_for_channels`` (``src/cpu/model.rs:1648-1673``): (ci, co, stride)."""
    return [
        [(c1, c1, (1, 1)), (c1, c1, (1, 1))],
        [(c1, c2, (2, 2)), (c2, c2, (1, 1)), (c2, c2, (1, 1))],
        [(c2, c3, (2, 2))] + [(c3, c3, (1, 1))] * 4,
        [(c3, c4, (2, 2)), (c4, c4, (1, 1)), (c4, c4, (1, 1))],
    ]


def recognizer_stage_specs(size):
    """``recognizer_stages`` / ``small_`` / ``tiny_`` (``src/cpu/model.rs:2057-2122``)."""
    if size == "medium":
        return [[(128, 128, (1, 1))],
                [(128, 256, (1, 1)), (256, 256, (1, 1)), (256, 256, (1, 1))],
                [(256, 512, (2, 1))] + [(512, 512, (1, 1))] * 6,
                [(512, 768, (2, 1)), (768, 768, (1, 1)), (768, 768, (1, 1))]]
    if size == "small":
        return [[(96, 96, (1, 1))],
                [(96, 96, (1, 1)), (96, 96, (1, 1))],
                [(96, 192, (2, 1))] + [(192, 192, (1, 1))] * 6,
                [(192, 384, (2, 1)), (384, 384, (1, 1)), (384, 384, (1, 1))]]
    return [[(48, 48, (1, 1))],
            [(48, 48, (1, 1))],
            [(48, 96, (2, 1)), (96, 96, (1, 1)), (96, 96, (1, 1))],
            [(96, 160, (2, 1)), (160, 160, (1, 1)), (160, 160, (1, 1)), (160, 160, (1, 1))]]


def backbone(wt, x, specs, small=False):
    """``LcNetBackbone::forward`` (``src/cpu/model.rs:800-808``): every stage's output."""
    h = _t("stem", small_stem(wt, x) if small else large_stem(wt, x))
    outs = []
    for s, stage in enumerate(specs):
        for b, (ci, co, stride) in enumerate(stage):
            h = _t(f"block{s}.{b}",
                   lcnet_block(wt, f"model.backbone.encoder.blocks.{s}.blocks.{b}", h, ci, co, stride))
        outs.append(h)
    return outs


# ---------------------------------------------------------------- necks
def variant_se_gate(wt, prefix, x):
    """``VariantSqueezeExcitation::attention`` (``src/cpu/model.rs:1100-1104``): hsig(1/5)."""
    pooled = x.mean(dim=(2, 3), keepdim=True)
    r = F.relu(conv(wt, f"{prefix}.conv1", pooled, bias=True))
    return hard_sigmoid(conv(wt, f"{prefix}.conv2", r, bias=True), 0.2)


def rep_lk_fpn(wt, stages, k):
    """``RepLkFpn::forward`` (``src/cpu/model.rs:1234-1253``) with
    ``ResidualSqueezeExcitation`` (``:1138-1142``) and
    ``DepthwiseSeparableConv`` (``:1185-1194``); ``into_residual_mul`` is
    ``x + x * g`` (``src/cpu/backend.rs:180-199``)."""
    fused = []
    for i, f in enumerate(stages):
        h = conv(wt, f"model.neck.insert_conv.{i}.in_conv", f)
        g = variant_se_gate(wt, f"model.neck.insert_conv.{i}.squeeze_excitation_block", h)
        fused.append(_t(f"fpn.insert{i}", h + h * g))
    for i in (2, 1, 0):  # top-down: the level above is already updated
        fused[i] = fused[i] + nearest_up(fused[i + 1], 2)
    feats = []
    for i, f in enumerate(fused):
        p = f"model.neck.input_conv.{i}"
        c = f.shape[1]
        h = conv(wt, f"{p}.depthwise_convolution", f, pads=(k // 2,) * 4, groups=c, bias=True)
        h = conv(wt, f"{p}.pointwise_convolution", h)
        g = variant_se_gate(wt, f"{p}.squeeze_excitation_module", h)
        feats.append(_t(f"fpn.feature{i}", h + h * g))
    feats = feats[::-1]  # deepest first
    return torch.cat([nearest_up(f, s) for f, s in zip(feats, (8, 4, 2, 1))], dim=1)


def intraclass_block(wt, prefix, x):
    """``IntraclassBlock::forward`` (``src/cpu/model.rs:939-945``) with the
    three branches of each ratio run separately and summed."""
    r = conv(wt, f"{prefix}.conv_reduce_channel", x, bias=True)
    for ratio, k in (("longratio", 7), ("midratio", 5), ("shortratio", 3)):
        p = k // 2
        sym = conv(wt, f"{prefix}.symmetric_conv_long_{ratio}", r, pads=(p, p, p, p), bias=True)
        ver = conv(wt, f"{prefix}.vertical_long_to_small_conv_{ratio}", r, pads=(p, 0, p, 0), bias=True)
        hor = conv(wt, f"{prefix}.horizontal_small_to_long_conv_{ratio}", r, pads=(0, p, 0, p), bias=True)
        r = sym + ver + hor
    return x + conv_bn_act(wt, f"{prefix}.conv_final", r, bias=True, norm="norm", act="relu")


def medium_neck(wt, stages):
    """``DetectorNeck::forward`` (``src/cpu/model.rs:1021-1066``); the rank-one
    9x9 convolutions run dense on the stored weights."""
    n = "model.neck"
    adj = [conv(wt, f"{n}.input_channel_adjustment_convolution.{i}", f) for i, f in enumerate(stages)]
    td = [None] * 4
    td[3] = adj[3]
    for i in (2, 1, 0):
        td[i] = adj[i] + nearest_up(td[i + 1], 2)
    proj = [conv(wt, f"{n}.input_feature_projection_convolution.{i}", f, pads=(4, 4, 4, 4), bias=True)
            for i, f in enumerate(td)]
    bu = []
    for i, p in enumerate(proj):
        if bu:
            p = p + conv(wt, f"{n}.path_aggregation_head_convolution.{i - 1}", bu[-1], (2, 2), (1, 1, 1, 1))
        bu.append(_t(f"neck.bottom_up{i}", p))
    lat = [_t(f"neck.lateral{i}", conv(wt, f"{n}.path_aggregation_lateral_convolution.{i}", f, pads=(4, 4, 4, 4),
                                        bias=True))
           for i, f in enumerate(bu)]
    refined = [_t(f"neck.refined{i}", intraclass_block(wt, f"{n}.intraclass_blocks.{i}", f))
               for i, f in enumerate(lat)]
    refined = refined[::-1]
    return torch.cat([nearest_up(f, s) for f, s in zip(refined, (8, 4, 2, 1))], dim=1)


def detector_head(wt, x):
    """``DetectorHead::forward`` (``src/cpu/model.rs:1516-1520``): 3x3+BN+ReLU,
    2x2 s2 transposed conv + BN over its output channels + ReLU, 2x2 s2
    transposed conv to one channel + sigmoid."""
    d = _t("head.down", conv_bn_act(wt, "head.conv_down", x, pads=(1, 1, 1, 1), norm="norm", act="relu"))
    u = F.conv_transpose2d(d, wt("head.conv_up.convolution.weight"), wt("head.conv_up.convolution.bias"), stride=2)
    u = _t("head.up", F.relu(batch_norm(u, wt, "head.conv_up.norm")))
    f = F.conv_transpose2d(u, wt("head.conv_final.weight"), wt("head.conv_final.bias"), stride=2)
    return torch.sigmoid(f)


DETECTOR_CHANNELS = {"medium": (128, 256, 512, 896), "small": (48, 96, 192, 384), "tiny": (32, 48, 64, 160)}
FPN_KERNEL = {"small": 7, "tiny": 5}


def detector(wt, size, x):
    """``Detector::infer`` (``src/cpu/model.rs:1622-1625``): [N,3,H,W] -> [N,1,H,W]."""
    stages = backbone(wt, x, detector_stage_specs(*DETECTOR_CHANNELS[size]))
    neck = medium_neck(wt, stages) if size == "medium" else rep_lk_fpn(wt, stages, FPN_KERNEL[size])
    return detector_head(wt, _t("neck", neck))


# ---------------------------------------------------------------- recognizers
def linear(wt, prefix, x):
    return F.linear(x, wt(f"{prefix}.weight"), wt(f"{prefix}.bias"))


def layer_norm(wt, prefix, x):
    """``LayerNorm`` with eps 1e-6 (``src/cpu/model.rs:1683``)."""
    return F.layer_norm(x, (x.shape[-1],), wt(f"{prefix}.weight"), wt(f"{prefix}.bias"), eps=1e-6)


def rec_attention(wt, prefix, x, heads=8):
    """``RecAttention::forward`` (``src/cpu/model.rs:1703-1725``): qkv viewed as
    [B, T, 3, heads, hd], softmax(q k^T hd^-0.5) v, projection."""
    b, t, h = x.shape
    hd = h // heads
    qkv = linear(wt, f"{prefix}.qkv", x).reshape(b, t, 3, heads, hd).permute(2, 0, 3, 1, 4)
    q, k, v = qkv[0], qkv[1], qkv[2]
    w = torch.softmax(torch.matmul(q, k.transpose(2, 3)) * hd ** -0.5, dim=-1)
    o = torch.matmul(w, v).transpose(1, 2).reshape(b, t, h)
    return linear(wt, f"{prefix}.projection", o)


def rec_block(wt, prefix, x):
    """``RecBlock::forward`` (``src/cpu/model.rs:1768-1772``)."""
    o = x + rec_attention(wt, f"{prefix}.self_attn", layer_norm(wt, f"{prefix}.layer_norm1", x))
    m = linear(wt, f"{prefix}.mlp.fc2", F.silu(linear(wt, f"{prefix}.mlp.fc1", layer_norm(wt, f"{prefix}.layer_norm2", o))))
    return o + m


def rec_encoder(wt, x):
    """``RecEncoder::forward`` (``src/cpu/model.rs:1825-1842``): x [N, C, 1, T]
    -> [N, T, hidden]; the skip branch is added after the final LayerNorm."""
    e = "head.encoder"
    skip = _t("svtr.skip", conv_bn_act(wt, f"{e}.conv_block.0", x, act="silu"))
    h = conv_bn_act(wt, f"{e}.conv_block.1", x, act="silu")
    c = h.shape[1]
    h = _t("svtr.hidden", h + conv_bn_act(wt, f"{e}.conv_block.2", h, pads=(0, 3, 0, 3), groups=c, act="silu"))
    n, c, hh, ww = h.shape
    seq = h.flatten(2, 3).transpose(1, 2)
    for i in range(2):
        seq = _t(f"svtr.block{i}", rec_block(wt, f"{e}.svtr_block.{i}", seq))
    out = layer_norm(wt, f"{e}.norm", seq).reshape(n, hh, ww, c).permute(0, 3, 1, 2) + skip
    return _t("svtr.encoder", out.squeeze(2).transpose(1, 2))


def tiny_head(wt, x):
    """``TinyRecognizerHead::forward`` (``src/cpu/model.rs:1930-1935``) with
    ``Conv1dBn`` (``:1877-1911``) run as 1-D convolutions on [N, C, T]."""
    s = x.squeeze(2)
    h = F.conv1d(s, wt("head.conv1.weight"), padding=2, groups=160)
    h = F.hardswish(batch_norm(h, wt, "head.norm1"))
    _t("tiny.conv1", h.unsqueeze(2))
    h = F.conv1d(h, wt("head.conv2.weight"))
    h = F.hardswish(batch_norm(h, wt, "head.norm2"))
    _t("tiny.conv2", h.unsqueeze(2))
    seq = h.transpose(1, 2)
    return torch.softmax(linear(wt, "head.fc2", linear(wt, "head.fc1", seq)), dim=-1)


def recognizer(wt, size, x):
    """``Recognizer::infer`` (``src/cpu/model.rs:2034-2039``): [N,3,48,W] -> [N,T,V]."""
    stages = backbone(wt, x, recognizer_stage_specs(size), small=size == "tiny")
    pooled = _t("pool", F.avg_pool2d(stages[-1], (3, 2), (3, 2)))
    if size == "tiny":
        return tiny_head(wt, pooled)
    return torch.softmax(linear(wt, "head.head", rec_encoder(wt, pooled)), dim=-1)


def forward(kind, size, weights, x, trace=None):
    """Runs one model in float64; ``weights`` is a path or a ``{name: array}``
    dict.  With ``trace`` a dict, it receives the named intermediates."""
    global _TRACE
    wt = weights if isinstance(weights, Weights) else (
        Weights(weights) if isinstance(weights, dict) else Weights.load(weights))
    _TRACE = trace
    try:
        with torch.no_grad():
            xt = torch.from_numpy(np.asarray(x, dtype=np.float64))
            y = detector(wt, size, xt) if kind == "det" else recognizer(wt, size, xt)
    finally:
        _TRACE = None
    return y.numpy()
