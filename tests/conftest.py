"""Shared test setup: the `gpu` marker and helpers.

GPU tests run only with a visible ROCm device; on a machine with a GPU they
require the HIP library (no fallback path exists)."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm) device and the built HIP library")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:  # noqa: BLE001
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no ROCm device visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_terminal_summary(terminalreporter):
    """The full-size oracle checks' errors (tests/gpu_util.SUMMARY), one line each."""
    from tests import gpu_util
    if gpu_util.SUMMARY:
        terminalreporter.write_sep("-", "full-size workloads against the oracle (relative inf-norm errors)")
        for line in gpu_util.SUMMARY:
            terminalreporter.write_line(line)
