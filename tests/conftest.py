import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP) device")


# Files whose latest kernel changes have not yet passed on a GPU run after the others (the
# no-allocation test stays last), so that under -x a failure there does not hide the results
# of every file collected after it.
LATE_FILES = ("test_gpu_inference.py",)


def _order(item):
    name = os.path.basename(str(item.fspath))
    return (name == "test_zz_no_alloc.py", name in LATE_FILES)


def pytest_collection_modifyitems(config, items):
    items.sort(key=_order)  # stable: the order inside each group is unchanged
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no HIP device")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
