"""The postprocess entry point that allocates no device memory
(``ppocr_hip_db_postprocess_static``), against the allocating entry point
``ppocr_hip_db_postprocess`` on the same maps, through the C ABI.

Bars as the device postprocess tests (tests/test_postprocess_gpu.py): the
same number of detections per map, scores within 1e-6 (fp64 moments summed
in another order), polygons within 1e-2 source pixels.  Two calls in a row,
the second on a smaller batch, so a stale first-call scratch would show; a
request larger than the static scratch is rejected, and the next call works.
"""

import numpy as np
import pytest

import oracle
import ppocr_hip

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    g = ppocr_hip.Gpu(0)
    yield g
    g.close()


def blob_maps(seed, n, h, w, blobs=20):
    rng = np.random.default_rng(seed)
    maps = rng.random((n, h, w)).astype(np.float32) * 0.25
    for i in range(n):
        for _ in range(blobs):
            y0, x0 = rng.integers(0, h - 8), rng.integers(0, w - 8)
            hh, ww = rng.integers(3, 20), rng.integers(4, 60)
            maps[i, y0:y0 + hh, x0:x0 + ww] = rng.uniform(0.3, 1.0)
    return maps


def same(a, b):
    assert [len(d) for d in a] == [len(d) for d in b]
    for da, db in zip(a, b):
        for u, v in zip(da, db):
            assert abs(u.score - v.score) <= 1e-6
            assert np.abs(u.polygon - v.polygon).max() <= 1e-2


def test_static_postprocess_matches_allocating_entry_point(gpu):
    first = blob_maps(1, 3, 416, 736)
    tr1 = [(1472, 832, 736, 416), (736, 416, 700, 400), (368, 208, 736, 416)]
    second = blob_maps(2, 1, 160, 320, blobs=8)
    tr2 = [(320, 160, 320, 160)]
    for maps, tr in ((first, tr1), (second, tr2)):
        print(f"static postprocess: maps {maps.shape}", flush=True)
        want = gpu.db_postprocess(maps, tr)
        got = gpu.db_postprocess_static(maps, tr)
        same(got, want)
        assert sum(len(d) for d in got) > 0
        # and the oracle agrees on the counts
        for i in range(maps.shape[0]):
            _, scores, _ = oracle.extract_detections(maps[i], tr[i])
            assert len(got[i]) == len(scores)


def test_static_postprocess_rejects_maps_beyond_its_scratch(gpu):
    big = np.zeros((8, 416, 736), np.float32)
    with pytest.raises(ppocr_hip.GpuError) as e:
        gpu.db_postprocess_static(big, [(736, 416, 736, 416)] * 8)
    assert e.value.kind == "InvalidInput"
    maps = blob_maps(3, 2, 96, 128, blobs=5)
    tr = [(128, 96, 128, 96)] * 2
    same(gpu.db_postprocess_static(maps, tr), gpu.db_postprocess(maps, tr))


def _free_device_bytes():
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def test_static_postprocess_allocates_no_device_memory():
    """Device memory is unchanged across a static call on maps larger than
    any before it.  That the measure sees allocations of this size is shown
    by a device image of 24 MB held across a second reading."""
    g = ppocr_hip.Gpu(0)
    try:
        warm = blob_maps(4, 1, 64, 96, blobs=3)
        g.db_postprocess_static(warm, [(96, 64, 96, 64)])
        maps = blob_maps(5, 2, 416, 736)
        tr = [(736, 416, 736, 416)] * 2
        before = _free_device_bytes()
        got = g.db_postprocess_static(maps, tr)
        after_static = _free_device_bytes()
        image = g.upload_rgb(np.zeros((2000, 4000, 3), np.uint8))
        with_image = _free_device_bytes()
        image.close()
        print(f"free device bytes: {before} -> {after_static} (static call) -> {with_image} (24 MB image held)",
              flush=True)
        same(got, g.db_postprocess(maps, tr))
        assert after_static == before
        assert after_static - with_image >= 8 << 20
    finally:
        g.close()
