"""Pins the oracle's network composition (CPU only).

Every primitive of the oracle is pinned by known-answer tests elsewhere; this
file pins how the primitives are wired into the six networks
(``src/cpu/model.rs``), in three ways:

1. An independent float64 PyTorch functional model (``torch_reference.py``:
   unfolded batch norm, dense rank-one 9x9 weights, unfused intraclass
   branches, library primitives) agrees with the oracle on every traced
   intermediate (stem, every LCNet block, neck levels, head, encoder) and on
   the output, for all six tiers.
2. Constructed weights whose outputs the mathematics fixes: each check makes
   one module reduce to a closed form, so a wiring mistake there changes the
   value by far more than rounding (residual source, gate constants, concat
   order, BN fold axis, skip/LayerNorm order, attention layout, tiny head).
3. Planted mistakes: the oracle can plant one wiring mistake at a time
   (``enum Fault`` in oracle.cpp); each is shown to be caught, by the
   PyTorch comparison at the parity tolerance (1e-3) and, where one applies,
   by its closed-form check.

Bars: relative to each tensor's largest magnitude, traced intermediates
within 2e-5 of the float64 model (the oracle's float32 rounding measures
1e-6 to 2e-6 through the deepest network); detector maps within 5e-6 and
recognizer probabilities within 1e-4 (logits reach magnitude 35, so their
float32 rounding of ~4e-5 moves the softmax by up to ~3e-5).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
import seeded
import torch_reference as tr
from helpers import model_path

INTER_REL = 2e-5
DET_ABS = 5e-6
REC_ABS = 1e-4
PARITY_TOL = 1e-3

TIERS = [("det", "tiny"), ("det", "small"), ("det", "medium"), ("rec", "tiny"), ("rec", "small"), ("rec", "medium")]
DET_SHAPE = (1, 3, 64, 96)
REC_SHAPE = (2, 3, 48, 64)

# Names of the oracle's plantable mistakes, in ``enum Fault`` order, with the
# tiers on which each must be visible.
FAULTS = [
    ("lcnet_residual_from_block_input", [("det", "tiny")]),
    ("lcnet_se_gate_fifth", [("det", "tiny")]),
    ("neck_se_gate_sixth", [("det", "tiny")]),
    ("neck_concat_shallow_first", [("det", "tiny"), ("det", "medium")]),
    ("missing_gelu", [("det", "tiny")]),
    ("head_bn_input_axis", [("det", "tiny")]),
    ("svtr_skip_before_norm", [("rec", "small")]),
    ("recblock_residual_normed", [("rec", "small")]),
    ("qkv_head_major", [("rec", "small")]),
    ("tiny_head_no_hswish1", [("rec", "tiny")]),
    ("neck_se_plain_gate", [("det", "tiny")]),
    ("stem_concat_swapped", [("det", "tiny")]),
    ("intraclass_row_column_swapped", [("det", "medium")]),
    ("pan_from_projection", [("det", "medium")]),
    ("topdown_not_cascaded", [("det", "tiny"), ("det", "medium")]),
    ("attention_scale_hidden", [("rec", "small")]),
    ("small_stem_no_gelu", [("rec", "tiny")]),
]
FAULT_ID = {name: i + 1 for i, (name, _) in enumerate(FAULTS)}


class planted:
    """Context manager: plant oracle fault ``name`` (None = none)."""

    def __init__(self, name):
        self.fault = 0 if name is None else FAULT_ID[name]

    def __enter__(self):
        oracle.set_fault(self.fault)

    def __exit__(self, *exc):
        oracle.set_fault(0)


def _input(kind, seed=5):
    shape = DET_SHAPE if kind == "det" else REC_SHAPE
    return seeded.seeded_batch(shape[0], shape[2], shape[3], seed, detector=kind == "det")


def _oracle_run(kind, size, weights, x):
    """Oracle output and traced intermediates; ``weights`` is a path."""
    oracle.set_tracing(True)
    try:
        y = oracle.Model(kind, weights, size).forward(x)
        names = _traced_names(kind, size)
        inter = {n: oracle.traced(n) for n in names}
    finally:
        oracle.set_tracing(False)
    return y, inter


def _traced_names(kind, size):
    specs = (tr.detector_stage_specs(*tr.DETECTOR_CHANNELS[size]) if kind == "det"
             else tr.recognizer_stage_specs(size))
    names = ["stem"] + [f"block{s}.{b}" for s, st in enumerate(specs) for b in range(len(st))]
    if kind == "det":
        if size == "medium":
            names += [f"neck.{p}{i}" for p in ("bottom_up", "lateral", "refined") for i in range(4)]
        else:
            names += [f"fpn.{p}{i}" for p in ("insert", "feature") for i in range(4)]
        names += ["neck", "head.down", "head.up"]
    else:
        names += ["pool"]
        names += ["tiny.conv1", "tiny.conv2"] if size == "tiny" else [
            "svtr.skip", "svtr.hidden", "svtr.block0", "svtr.block1", "svtr.encoder"]
    return names


_REFERENCE = {}


def _reference(kind, size):
    """float64 model output and intermediates on the seeded weights (cached)."""
    key = (kind, size)
    if key not in _REFERENCE:
        trace = {}
        y = tr.forward(kind, size, model_path(kind, size), _input(kind), trace=trace)
        _REFERENCE[key] = (y, trace)
    return _REFERENCE[key]


def _output_diff(kind, size):
    y64, _ = _reference(kind, size)
    y, _ = _oracle_run(kind, size, model_path(kind, size), _input(kind))
    return float(np.abs(y - y64).max())


# ---------------------------------------------------------------- 1. independent model
@pytest.mark.parametrize("kind,size", TIERS)
def test_independent_model_matches_oracle(kind, size):
    y64, t64 = _reference(kind, size)
    y, inter = _oracle_run(kind, size, model_path(kind, size), _input(kind))
    assert y.shape == y64.shape
    for name, got in inter.items():
        want = t64[name]
        assert got.shape == want.shape, (name, got.shape, want.shape)
        rel = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
        assert rel <= INTER_REL, f"{kind} {size} {name}: relative difference {rel:.2e}"
    assert np.abs(y - y64).max() <= (DET_ABS if kind == "det" else REC_ABS)


def test_fault_table_matches_oracle():
    assert oracle.fault_count() == len(FAULTS) + 1


@pytest.mark.parametrize("name", [f for f, _ in FAULTS])
def test_planted_fault_is_caught_by_independent_model(name):
    tiers = dict(FAULTS)[name]
    with planted(name):
        diffs = [_output_diff(kind, size) for kind, size in tiers]
    assert min(diffs) > PARITY_TOL, f"fault {name} moves the output by only {diffs}"


# ---------------------------------------------------------------- 2. constructed weights
def _weights(kind, size):
    gain, head_gain = seeded.DEFAULT_GAINS[(kind, size)]
    return seeded.seeded_weights(kind, size, seed=11, gain=gain, head_gain=head_gain)


def _save(tmp_path, w, tag):
    from safetensors.numpy import save_file

    path = tmp_path / f"{tag}.safetensors"
    save_file({k: np.ascontiguousarray(v, dtype=np.float32) for k, v in w.items()}, str(path))
    return path


def _f32(v):
    return np.asarray(v, dtype=np.float32)


def _hard_sigmoid_fma(b, alpha):
    """clamp(fma(b, alpha, 0.5), 0, 1) in float32 for dyadic b (the float64
    product and sum are exact, so one rounding to float32 is the fma's)."""
    v = (np.asarray(b, np.float64) * np.float64(np.float32(alpha)) + 0.5).astype(np.float32)
    return np.clip(v, np.float32(0), np.float32(1))


def check_lcnet_residual_and_se_gate(tmp_path):
    """Tiny detector block 0.0 (32 -> 32, stride 1, with SE; residual).

    Token conv = identity (centre tap 1, bias 0); SE reduce = 0 so its ReLU
    is 0 and the gate is hard-sigmoid(x/6 + 0.5) of the expand bias b_c;
    channel_conv2's BN gamma and beta = 0, so the pair adds exactly 0.  The
    block output is then exactly x * g_c with x the stem output: taking the
    residual from the block input would give x + 0, a 1/5 gate other values.
    (src/cpu/model.rs:487-492, :591-602; src/cpu/backend.rs:470-477)
    """
    w = _weights("det", "tiny")
    p = "model.backbone.encoder.blocks.0.blocks.0"
    tok = np.zeros((32, 1, 3, 3), np.float32)
    tok[:, 0, 1, 1] = 1
    w[f"{p}.token_conv.weight"] = tok
    w[f"{p}.token_conv.bias"] = np.zeros(32, np.float32)
    w[f"{p}.token_squeeze_excitation.convolutions.0.weight"][:] = 0
    w[f"{p}.token_squeeze_excitation.convolutions.0.bias"][:] = 0
    b = _f32((np.arange(32) - 16) / 4.0)  # -4 .. 3.75: both clamps and the linear part
    w[f"{p}.token_squeeze_excitation.convolutions.2.bias"] = b
    w[f"{p}.channel_conv2.normalization.weight"][:] = 0
    w[f"{p}.channel_conv2.normalization.bias"][:] = 0
    _, inter = _oracle_run("det", "tiny", _save(tmp_path, w, "lcnet"), _input("det"))
    x = inter["stem"]
    g = _hard_sigmoid_fma(b, 1.0 / 6.0)
    want = x * g[None, :, None, None]
    return np.array_equal(inter["block0.0"], want)


def check_neck_se_gate(tmp_path):
    """Tiny detector FPN insert level 0: h = in_conv(stage 0); SE conv1 = 0, so
    the gate is hard-sigmoid(x/5 + 0.5) of conv2's bias; the output is
    h + h * g (src/cpu/model.rs:1100-1104, :1138-1142)."""
    w = _weights("det", "tiny")
    p = "model.neck.insert_conv.0.squeeze_excitation_block"
    w[f"{p}.conv1.weight"][:] = 0
    w[f"{p}.conv1.bias"][:] = 0
    b = _f32((np.arange(64) - 32) / 6.0 * 1.0)
    b = _f32(np.round(b * 8) / 8)  # dyadic
    w[f"{p}.conv2.bias"] = b
    _, inter = _oracle_run("det", "tiny", _save(tmp_path, w, "neckse"), _input("det"))
    x = inter["block0.1"].astype(np.float64)
    h = np.einsum("oc,nchw->nohw", w["model.neck.insert_conv.0.in_conv.weight"][:, :, 0, 0].astype(np.float64), x)
    g = _hard_sigmoid_fma(b, 0.2).astype(np.float64)[None, :, None, None]
    want = h + h * g
    got = inter["fpn.insert0"]
    return np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def check_fpn_concat_deepest_first(tmp_path):
    """Tiny detector FPN: each level's depthwise conv has zero weights and bias
    c_i = (i + 1) / 4, the pointwise weights are 1/64 and the SE gate is 0.5,
    so level i is the constant 1.5 c_i exactly; the neck output's channel
    block j must hold level 3 - j (deepest first, src/cpu/model.rs:1251-1252)."""
    w = _weights("det", "tiny")
    for i in range(4):
        p = f"model.neck.input_conv.{i}"
        w[f"{p}.depthwise_convolution.weight"][:] = 0
        w[f"{p}.depthwise_convolution.bias"][:] = (i + 1) / 4.0
        w[f"{p}.pointwise_convolution.weight"][:] = 1.0 / 64.0
        w[f"{p}.squeeze_excitation_module.conv1.weight"][:] = 0
        w[f"{p}.squeeze_excitation_module.conv1.bias"][:] = 0
        w[f"{p}.squeeze_excitation_module.conv2.bias"][:] = 0
    _, inter = _oracle_run("det", "tiny", _save(tmp_path, w, "fpncat"), _input("det"))
    neck = inter["neck"]
    want = np.concatenate([np.full((1, 16) + neck.shape[2:], 1.5 * (4 - j) / 4.0, np.float32) for j in range(4)], 1)
    return np.array_equal(neck, want)


def check_medium_concat_deepest_first(tmp_path):
    """Medium detector neck: each lateral rank-one conv has zero weights and
    bias c_i, each intraclass block's conv_final BN has gamma = beta = 0
    (so the block adds 0), so refined level i is the constant c_i; the concat
    must hold level 3 - j in channel block j (src/cpu/model.rs:1064-1065)."""
    w = _weights("det", "medium")
    for i in range(4):
        w[f"model.neck.path_aggregation_lateral_convolution.{i}.weight"][:] = 0
        w[f"model.neck.path_aggregation_lateral_convolution.{i}.bias"][:] = (i + 1) / 4.0
        q = f"model.neck.intraclass_blocks.{i}.conv_final.norm"
        w[f"{q}.weight"][:] = 0
        w[f"{q}.bias"][:] = 0
    _, inter = _oracle_run("det", "medium", _save(tmp_path, w, "medcat"), _input("det"))
    neck = inter["neck"]
    want = np.concatenate([np.full((1, 64) + neck.shape[2:], (4 - j) / 4.0, np.float32) for j in range(4)], 1)
    return np.array_equal(neck, want)


def check_head_bn_output_axis(tmp_path):
    """Tiny detector head conv_up ([in 16, out 16, 2, 2], IOHW): weights route
    input channel i to output channel i + 1 (mod 16) at every tap, bias 0;
    its BN has gamma_o = 0.5 + o/32, beta = mean = 0, var = 1.  The fold
    scales output channels (src/cpu/model.rs:1440-1477), so
    up[o, 2y+ky, 2x+kx] = relu(down[o-1, y, x] * s_o) exactly."""
    w = _weights("det", "tiny")
    W = np.zeros((16, 16, 2, 2), np.float32)
    for i in range(16):
        W[i, (i + 1) % 16] = 1
    w["head.conv_up.convolution.weight"] = W
    w["head.conv_up.convolution.bias"] = np.zeros(16, np.float32)
    gamma = _f32(0.5 + np.arange(16) / 32.0)
    w["head.conv_up.norm.weight"] = gamma
    w["head.conv_up.norm.bias"] = np.zeros(16, np.float32)
    w["head.conv_up.norm.running_mean"] = np.zeros(16, np.float32)
    w["head.conv_up.norm.running_var"] = np.ones(16, np.float32)
    _, inter = _oracle_run("det", "tiny", _save(tmp_path, w, "headbn"), _input("det"))
    d = inter["head.down"]
    s = gamma / np.sqrt(np.float32(1) + np.float32(1e-5))
    up = np.roll(d, 1, axis=1) * s[None, :, None, None]
    want = np.maximum(np.repeat(np.repeat(up, 2, axis=2), 2, axis=3), 0)
    return np.array_equal(inter["head.up"], want)


def _svtr_identity_blocks(w, blocks=(0, 1)):
    for i in blocks:
        p = f"head.encoder.svtr_block.{i}"
        for leaf in ("self_attn.projection", "mlp.fc2"):
            w[f"{p}.{leaf}.weight"][:] = 0
            w[f"{p}.{leaf}.bias"][:] = 0


def _layer_norm64(x, weight, bias, eps=1e-6):
    x = x.astype(np.float64)
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + eps) * weight.astype(np.float64) + bias.astype(np.float64)


def check_svtr_skip_after_norm(tmp_path):
    """Small recognizer encoder: both LightSVTR blocks reduce to the identity
    (projection and fc2 zero), so the encoder output is LN(seq) + skip with
    seq the reduce + local tensor; the skip is added after the final
    LayerNorm (src/cpu/model.rs:1825-1842)."""
    w = _weights("rec", "small")
    _svtr_identity_blocks(w)
    _, inter = _oracle_run("rec", "small", _save(tmp_path, w, "svtrskip"), _input("rec"))
    seq = inter["svtr.hidden"][:, :, 0, :].transpose(0, 2, 1)
    skip = inter["svtr.skip"][:, :, 0, :].transpose(0, 2, 1)
    if not np.array_equal(inter["svtr.block1"], seq):
        return False
    want = _layer_norm64(seq, w["head.encoder.norm.weight"], w["head.encoder.norm.bias"]) + skip
    got = inter["svtr.encoder"]
    return np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def check_attention_layout(tmp_path):
    """Small recognizer block 0: LN1 = plain normalisation, the query third
    of qkv is zero (uniform softmax), the value third is the identity, the
    projection is the identity and fc2 zero; the block output is then
    x + mean_t(LN(x)) at every step.  This fixes the residual source
    (x, not LN(x)) and the qkv split [3, heads, hd] (src/cpu/model.rs:1703-1725,
    :1768-1772)."""
    w = _weights("rec", "small")
    h = 120
    p = "head.encoder.svtr_block.0"
    w[f"{p}.layer_norm1.weight"][:] = 1
    w[f"{p}.layer_norm1.bias"][:] = 0
    qkv = w[f"{p}.self_attn.qkv.weight"]
    qkv[:h] = 0
    qkv[2 * h:] = np.eye(h, dtype=np.float32)
    w[f"{p}.self_attn.qkv.bias"][:] = 0
    w[f"{p}.self_attn.projection.weight"] = np.eye(h, dtype=np.float32)
    w[f"{p}.self_attn.projection.bias"][:] = 0
    w[f"{p}.mlp.fc2.weight"][:] = 0
    w[f"{p}.mlp.fc2.bias"][:] = 0
    _, inter = _oracle_run("rec", "small", _save(tmp_path, w, "attn"), _input("rec"))
    x = inter["svtr.hidden"][:, :, 0, :].transpose(0, 2, 1).astype(np.float64)
    ln = _layer_norm64(x, np.ones(h), np.zeros(h))
    want = x + ln.mean(1, keepdims=True)
    got = inter["svtr.block0"]
    return np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


def _hardswish64(x):
    return x * np.clip(x / 6.0 + 0.5, 0.0, 1.0)


def check_tiny_head(tmp_path):
    """Tiny recognizer head with conv1 = identity depthwise tap, conv2 =
    identity, BN statistics (1, 0, 0, 1): the output is
    softmax(fc2(fc1(hswish(hswish(pool * s) * s)^T))) with s = 1/sqrt(1 + 1e-5)
    (src/cpu/model.rs:1877-1936)."""
    w = _weights("rec", "tiny")
    c1 = np.zeros((160, 1, 5), np.float32)
    c1[:, 0, 2] = 1
    w["head.conv1.weight"] = c1
    w["head.conv2.weight"] = np.eye(160, dtype=np.float32)[:, :, None]
    for n in ("head.norm1", "head.norm2"):
        w[f"{n}.weight"][:] = 1
        w[f"{n}.bias"][:] = 0
        w[f"{n}.running_mean"][:] = 0
        w[f"{n}.running_var"][:] = 1
    y, inter = _oracle_run("rec", "tiny", _save(tmp_path, w, "tinyhead"), _input("rec"))
    s = 1.0 / np.sqrt(1.0 + 1e-5)
    pool = inter["pool"][:, :, 0, :].astype(np.float64)
    h = _hardswish64(_hardswish64(pool * s) * s).transpose(0, 2, 1)
    f1 = h @ w["head.fc1.weight"].astype(np.float64).T + w["head.fc1.bias"]
    logits = f1 @ w["head.fc2.weight"].astype(np.float64).T + w["head.fc2.bias"]
    e = np.exp(logits - logits.max(-1, keepdims=True))
    want = e / e.sum(-1, keepdims=True)
    return np.abs(y - want).max() <= REC_ABS


CHECKS = {
    "lcnet_residual_and_se_gate": (check_lcnet_residual_and_se_gate,
                                   ["lcnet_residual_from_block_input", "lcnet_se_gate_fifth"]),
    "neck_se_gate": (check_neck_se_gate, ["neck_se_gate_sixth", "neck_se_plain_gate"]),
    "fpn_concat_deepest_first": (check_fpn_concat_deepest_first, ["neck_concat_shallow_first"]),
    "medium_concat_deepest_first": (check_medium_concat_deepest_first, ["neck_concat_shallow_first"]),
    "head_bn_output_axis": (check_head_bn_output_axis, ["head_bn_input_axis"]),
    "svtr_skip_after_norm": (check_svtr_skip_after_norm, ["svtr_skip_before_norm"]),
    "attention_layout": (check_attention_layout, ["recblock_residual_normed", "qkv_head_major"]),
    "tiny_head": (check_tiny_head, ["tiny_head_no_hswish1"]),
}


@pytest.mark.parametrize("check", sorted(CHECKS))
def test_constructed_weights_closed_form(check, tmp_path):
    fn, _ = CHECKS[check]
    assert fn(tmp_path)


@pytest.mark.parametrize("check,fault", [(c, f) for c in sorted(CHECKS) for f in CHECKS[c][1]])
def test_planted_fault_breaks_closed_form(check, fault, tmp_path):
    fn, _ = CHECKS[check]
    with planted(fault):
        assert not fn(tmp_path), f"closed-form check {check} does not see fault {fault}"
