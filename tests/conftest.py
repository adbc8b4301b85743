"""Test set-up: import paths, the `gpu` marker, and shared helpers."""
import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "3dgs-project_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libamdsplat.so")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_runtest_setup(item):
    # name the case before it runs, so a GPU failure can be attributed from partial output
    if "gpu" in item.keywords and os.environ.get("AMDSPLAT_TRACE_TESTS", "1") == "1":
        print(f"\n[gpu-test] {item.nodeid}", flush=True)


def pytest_terminal_summary(terminalreporter):
    """The numbers parity tests record with record_property("parity", line) (per-parameter
    end-to-end errors, the chain's amplification, ambiguous-pixel counts), printed after the
    run even under -q, in the order the tests ran."""
    lines = []
    for key in ("passed", "failed"):
        for rep in terminalreporter.stats.get(key, []):
            for name, value in getattr(rep, "user_properties", ()):
                if name == "parity":
                    lines.append((rep.nodeid, value))
    if lines:
        terminalreporter.section("parity numbers")
        for nodeid, value in lines:
            terminalreporter.write_line(f"{value}")
