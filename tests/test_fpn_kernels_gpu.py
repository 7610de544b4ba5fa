"""Kernel-level checks of the FPN's batched launches on the GPU.

The RepLk FPN of the tiny and small detectors forms four per-level
squeeze-excitation gates after its insert convs and four more after its
input convs, and writes every level's x + x*g upsampled into its concat
slot (src/cpu/model.rs:1069-1105, :1138-1142, :1188-1254).  The plans run
each group as one launch: se_multi_kernel (one workgroup row per gate, from
the channel sums the producing convs left) and gate_residual_multi_kernel
(each block finds its level).  Both run here through libppocr_hip_probe.so
and are compared with float64: gate = clamp(v / 5 + 1/2, 0, 1) of
v = W2 relu(W1 mean + b1) + b2, mean = (sum of the partial rows) / HW; and
out = x + x*g, replicated rep x rep.
"""
import ctypes

import numpy as np
import pytest

from test_conv_kernels_gpu import PROBE, _ptr

pytestmark = pytest.mark.gpu

ACT_HSIG5 = 5


def _lib():
    if not PROBE.exists():
        raise RuntimeError(f"{PROBE} is not built (make -C ppocr-rs_amd)")
    lib = ctypes.CDLL(str(PROBE))
    f = ctypes.POINTER(ctypes.c_float)
    ip = ctypes.POINTER(ctypes.c_int)
    i = ctypes.c_int
    lib.ppocr_probe_se_multi.argtypes = [i, i, ip, f, f, f, f, f, i, f]
    lib.ppocr_probe_se_multi.restype = i
    lib.ppocr_probe_gate_residual_multi.argtypes = [i, i, ip, f, f, f]
    lib.ppocr_probe_gate_residual_multi.restype = i
    return lib


def _ints(v):
    return (ctypes.c_int * len(v))(*v)


def _cat(arrays):
    return np.ascontiguousarray(np.concatenate([a.ravel() for a in arrays]).astype(np.float32))


# (n, [(HW, C, P, Cr) per gate]): the tiny detector's insert-conv gates
# (64 channels over 19136 .. 299 pixels, four column sums per 64-row tile)
# and input-conv gates (16 channels), two images, and a single gate.
SE_CASES = [
    ("insert convs", 1, [(19136, 64, 1196, 16), (4784, 64, 300, 16), (1196, 64, 76, 16), (299, 64, 20, 16)]),
    ("input convs", 1, [(19136, 16, 1196, 4), (4784, 16, 300, 4), (1196, 16, 76, 4), (299, 16, 20, 4)]),
    ("two images, three gates", 2, [(900, 32, 57, 8), (225, 32, 15, 8), (64, 32, 4, 8)]),
    ("one gate", 1, [(4000, 128, 250, 32)]),
    # Gates over 256 channels (or 64 reduced ones) whose weights still fit one
    # workgroup take the general body (se_multi_kind 2).
    ("general body", 2, [(4000, 512, 250, 32), (1000, 384, 63, 32)]),
]


@pytest.mark.parametrize("name,n,dims", SE_CASES, ids=[c[0] for c in SE_CASES])
def test_se_multi_matches_float64(name, n, dims):
    lib = _lib()
    rng = np.random.default_rng(7)
    parts, w1s, b1s, w2s, b2s, want = [], [], [], [], [], []
    for hw, c, p, cr in dims:
        part = rng.normal(0.0, 2.0, (n, p, c)).astype(np.float32)
        w1 = rng.normal(0.0, 0.3, (cr, c)).astype(np.float32)
        b1 = rng.normal(0.0, 0.1, cr).astype(np.float32)
        w2 = rng.normal(0.0, 0.3, (c, cr)).astype(np.float32)
        b2 = rng.normal(0.0, 0.1, c).astype(np.float32)
        mean = part.astype(np.float64).sum(axis=1) / hw
        hid = np.maximum(mean @ w1.T.astype(np.float64) + b1, 0.0)
        v = hid @ w2.T.astype(np.float64) + b2
        want.append(np.clip(v / 5.0 + 0.5, 0.0, 1.0))
        parts.append(part), w1s.append(w1), b1s.append(b1), w2s.append(w2), b2s.append(b2)
    flat = [d for g in dims for d in g]
    gates = np.zeros(sum(n * g[1] for g in dims), np.float32)
    rc = lib.ppocr_probe_se_multi(len(dims), n, _ints(flat), _ptr(_cat(parts)), _ptr(_cat(w1s)), _ptr(_cat(b1s)),
                                  _ptr(_cat(w2s)), _ptr(_cat(b2s)), ACT_HSIG5, _ptr(gates))
    assert rc == 0
    np.testing.assert_allclose(gates, np.concatenate([w.ravel() for w in want]), rtol=0, atol=2e-6)


def test_se_multi_refuses_mixed_kinds():
    # A 16-channel gate (small-weight body, kind 1) and a 384-channel one with
    # 32 hidden units (the general one-workgroup body, kind 2) cannot share a
    # launch; each alone can.
    lib = _lib()
    z = lambda k: np.zeros(k, np.float32)  # noqa: E731

    def run(dims):
        flat = [d for g in dims for d in g]
        part = sum(p * c for _, c, p, _ in dims)
        w = sum(c * cr for _, c, _, cr in dims)
        return lib.ppocr_probe_se_multi(len(dims), 1, _ints(flat), _ptr(z(part)), _ptr(z(w)),
                                        _ptr(z(sum(cr for *_, cr in dims))), _ptr(z(w)),
                                        _ptr(z(sum(c for _, c, _, _ in dims))), ACT_HSIG5,
                                        _ptr(z(sum(c for _, c, _, _ in dims))))

    small, general = (100, 16, 4, 4), (100, 384, 4, 32)
    assert run([small, general]) == 2
    assert run([general, small]) == 2
    assert run([small]) == 0
    assert run([general]) == 0


# (n, [(H, W, C, rep) per level]): the FPN's input-conv outputs into the
# concat slots (deepest level upsampled 8x), and odd sides.
GR_CASES = [
    ("fpn levels", 1, [(104, 184, 16, 1), (52, 92, 16, 2), (26, 46, 16, 4), (13, 23, 16, 8)]),
    ("two images, odd sides", 2, [(9, 13, 8, 1), (5, 7, 12, 3)]),
]


@pytest.mark.parametrize("name,n,dims", GR_CASES, ids=[c[0] for c in GR_CASES])
def test_gate_residual_multi_matches_float64(name, n, dims):
    lib = _lib()
    rng = np.random.default_rng(11)
    xs, gs, want = [], [], []
    for h, w, c, rep in dims:
        x = rng.normal(0.0, 1.0, (n, h, w, c)).astype(np.float32)
        g = rng.uniform(0.0, 1.0, (n, c)).astype(np.float32)
        y = x.astype(np.float64) + x.astype(np.float64) * g[:, None, None, :]
        want.append(np.repeat(np.repeat(y, rep, axis=1), rep, axis=2))
        xs.append(x), gs.append(g)
    flat = [d for g in dims for d in g]
    out = np.full(sum(a.size for a in want), np.nan, np.float32)
    rc = lib.ppocr_probe_gate_residual_multi(len(dims), n, _ints(flat), _ptr(_cat(xs)), _ptr(_cat(gs)), _ptr(out))
    assert rc == 0
    np.testing.assert_allclose(out, np.concatenate([w.ravel() for w in want]), rtol=2e-7, atol=1e-7)
