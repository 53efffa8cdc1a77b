import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "clef-hrx_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    # The library must match the sources: its embedded build identity is
    # compared with the tree's hash and a missing or stale library is rebuilt
    # from scratch (timestamps do not survive every copy of the tree). The
    # oracle's incremental make is a no-op when it is up to date.
    import build_id

    problem = build_id.stale()
    if problem:
        print(f"conftest: {problem}; rebuilding", flush=True)
        subprocess.run(["make", "-s", "-B", "-j", "16", "-C", PKG], check=True)
        problem = build_id.stale()
        assert problem is None, problem
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


def pytest_collection_modifyitems(config, items):
    # GPU tests need a visible device; on a CPU-only host they are skipped
    # rather than failing when the marker filter is not given.
    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover - torch import failure
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
