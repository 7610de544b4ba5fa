import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for sub in ("ppocr-rs_amd", "oracle"):
    p = str(ROOT / sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
