"""Test configuration: the `gpu` marker, import paths, build-on-demand."""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "llm-inference-cpp_amd")
sys.path.insert(0, ROOT)
sys.path.insert(0, PKG)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    # Build only when nothing is built yet; a fresh build is
    # __graft_entry__.build()'s job.
    need = [os.path.join(PKG, "libllmi_hip.so"), os.path.join(ROOT, "oracle", "liboracle.so")]
    if not all(os.path.exists(p) for p in need):
        import __graft_entry__

        __graft_entry__.build()


@pytest.fixture(scope="session")
def golden():
    import json

    import numpy as np

    with open(os.path.join(GOLDEN, "golden.json")) as f:
        rec = json.load(f)
    arrays = {}
    for name in ("quant_small", "shapes", "kernels", "tiny_models"):
        with np.load(os.path.join(GOLDEN, name + ".npz")) as z:
            arrays[name] = {k: z[k] for k in z.files}
    return rec, arrays
