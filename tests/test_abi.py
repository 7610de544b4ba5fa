"""The C-ABI library loads and exports every entry point include/ppocr_hip.h
declares; argument checks run before any device work (no GPU needed)."""

import ctypes
import pathlib
import re

import pytest

import ppocr_hip

ROOT = pathlib.Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "ppocr_hip.h").read_text()
    return sorted(set(re.findall(r"\b(ppocr_\w+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(ppocr_hip.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = ppocr_hip.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name


def test_null_arguments_are_rejected_without_device_work():
    lib = ppocr_hip.lib()
    assert lib.ppocr_hip_create(0, None) == 10  # InvalidInput
    assert b"null" in lib.ppocr_hip_last_error()
    shape = (ctypes.c_size_t * 4)()
    rank = ctypes.c_size_t()
    assert lib.ppocr_hip_output_shape(None, shape, ctypes.byref(rank)) == 10
    assert lib.ppocr_hip_forward(None, None, 0, None, 0) == 10
    assert lib.ppocr_hip_device_info(None, None) == 10


def test_gpu_info_struct_layout_matches_the_header():
    # char[256] + char[16] + char[64] + 4 ints + size_t (8-aligned)
    assert ctypes.sizeof(ppocr_hip.GpuInfoStruct) == 256 + 16 + 64 + 4 * 4 + 8
    assert ppocr_hip.GpuInfoStruct.total_memory.offset == 352


def test_missing_device_reports_a_gpu_error():
    try:
        g = ppocr_hip.Gpu(0)
    except ppocr_hip.GpuError as e:
        assert e.kind == "Gpu"
    else:  # running on a GPU machine
        g.close()


def test_status_names_follow_the_reference_error_enum():
    # src/gpu/error.rs:9-45, in declaration order after Ok.
    assert [ppocr_hip.STATUS[i] for i in range(1, 12)] == [
        "ReadFile", "Safetensors", "TensorNotFound", "UnsupportedDtype", "ShapeMismatch",
        "TensorSizeOverflow", "TensorByteLength", "InvalidTensorRange", "InvalidModel", "InvalidInput", "Gpu"]


@pytest.mark.parametrize("kind,size,count", [
    ("det", "tiny", 271), ("det", "small", 271), ("det", "medium", 350),
    ("rec", "tiny", 150), ("rec", "small", 250), ("rec", "medium", 269),
])
def test_seeded_schema_matches_reference_tensor_counts(kind, size, count):
    # src/gpu/model.rs:11-16
    import seeded

    assert len(seeded.schema(kind, size)) == count
