import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "yolo11.cu_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run on the GPU box)")


@pytest.fixture(scope="session")
def models(tmp_path_factory):
    """Lazily generated model dirs keyed by (arch, scale, task, cls_bias)."""
    import modelgen

    base = tmp_path_factory.mktemp("models")
    cache = {}

    def get(arch="yolo11", scale="n", task="detect", cls_bias=-8.0, imgsz=640, seed=0, nc=80):
        key = (arch, scale, task, cls_bias, imgsz, seed, nc)
        if key not in cache:
            d = str(base / "_".join(str(k) for k in key))
            modelgen.write_model(d, arch, scale, task, nc, imgsz, seed, cls_bias)
            cache[key] = d
        return cache[key]

    return get
