"""Host packing of the bf16 matrix-core depthwise taps (no GPU needed).

The table holds, per channel and tap row, the B operand of a 16x16x32
product as the matrix cores read it: lane l supplies B[k][n] for
k = 8 * (l // 16) + i (i = 0..7) and n = l % 16.  Multiplying a 32-column
input row segment by that B must give the depthwise correlation of the row
with the (bf16-rounded) taps at 16 consecutive output columns, exactly.
"""
import ctypes

import numpy as np

from test_conv_kernels_gpu import PROBE, bf16_round


def _table(w):
    lib = ctypes.CDLL(str(PROBE))
    lib.ppocr_probe_depthwise_table.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_int, ctypes.c_int,
                                                ctypes.POINTER(ctypes.c_uint16)]
    lib.ppocr_probe_depthwise_table.restype = None
    c, k, _ = w.shape
    out = np.zeros((c, k, 64, 8), np.uint16)
    w = np.ascontiguousarray(w, np.float32)
    lib.ppocr_probe_depthwise_table(w.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), c, k,
                                    out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)))
    return (out.astype(np.uint32) << 16).view(np.float32)


def test_packed_taps_multiply_to_the_correlation():
    rng = np.random.default_rng(3)
    for k in (5, 7, 9):
        c = 3
        w = rng.uniform(-1, 1, (c, k, k)).astype(np.float32)
        tab = _table(w)
        wb = bf16_round(w).astype(np.float64)
        for ch in range(c):
            for ky in range(k):
                b = np.zeros((32, 16))
                for lane in range(64):
                    for i in range(8):
                        b[8 * (lane // 16) + i, lane % 16] = tab[ch, ky, lane, i]
                # Input columns past 16 + k - 1 meet zero weights (the kernel
                # stores zeros there; any finite value gives the same sums).
                a = bf16_round(rng.uniform(-1, 1, 32).astype(np.float32)).astype(np.float64)
                got = a @ b
                want = np.array([sum(a[x + j] * wb[ch, ky, j] for j in range(k)) for x in range(16)])
                assert np.array_equal(got, want), (k, ch, ky)
                assert not b[16 + k - 1:].any()
