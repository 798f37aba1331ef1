import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def _build_library_if_absent():
    """Test modules import flydsl_amd, which loads libpa_fp8.so at import time.  Build it
    (hipcc cross-compiles without a GPU) only when nothing is built yet; the recipe is
    loaded by path because importing it through the package would load the library."""
    import importlib.util

    spec = importlib.util.spec_from_file_location("_flydsl_amd_build", os.path.join(ROOT, "flydsl_amd", "build.py"))
    fbuild = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(fbuild)
    if not fbuild.LIB_PATH.exists():
        fbuild.build()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libpa_fp8.so")
    _build_library_if_absent()


def pytest_collection_modifyitems(config, items):
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
