"""Test configuration: import paths, the `gpu` marker, an isolated candidate cache."""

import os
import sys
import tempfile
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "voodoo-dyn-quant_amd"))
sys.path.insert(0, str(ROOT))
os.environ.setdefault("VOODOO_CANDIDATE_CACHE_DIR", tempfile.mkdtemp(prefix="vq_test_cache_"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built libvoodoo_hip.so")


def pytest_report_header(config):
    return f"voodoo_quant tests; candidate cache at {os.environ['VOODOO_CANDIDATE_CACHE_DIR']}"
