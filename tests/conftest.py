import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# every chained scan call synchronises and checks the library's error mailbox
# (outside tests a failure is reported by the next chained call)
os.environ.setdefault("LTV_CHAIN_SYNC_CHECK", "1")
for p in (os.path.join(ROOT, "nanochat-filter_amd"), os.path.join(ROOT, "oracle"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def pytest_sessionfinish(session, exitstatus):
    """With LTV_ERR_REPORT=<path>, write every assert_close's error statistics
    (label, tolerance, max abs, normwise and element-wise relative error)."""
    path = os.environ.get("LTV_ERR_REPORT")
    if not path:
        return
    try:
        from ltv_test_utils import ERR_LOG
    except Exception:
        return
    import json
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "w") as fh:
        json.dump(ERR_LOG, fh, indent=0)
