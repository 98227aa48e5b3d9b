import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# measured parity errors of this session: (test id, quantity, error, bound)
_ERRORS = []


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (runs the HIP kernels through the C-ABI)")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        have_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        have_gpu = False
    if have_gpu:
        return
    skip = pytest.mark.skip(reason="no ROCm GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture
def record_error(request):
    """record_error(quantity, error, bound): keep a measured error for the session log.

    With EGNN_PARITY_LOG set, the session writes every recorded error to that
    path as JSON lines when it ends."""
    def rec(quantity, err, bound):
        _ERRORS.append(dict(test=request.node.nodeid, quantity=quantity, err=float(err), bound=float(bound)))
        print(f"[parity] {request.node.name} {quantity} {err:.3e} (bound {bound:.0e})", flush=True)
    return rec


def pytest_sessionfinish(session, exitstatus):
    path = os.environ.get("EGNN_PARITY_LOG")
    if not path or not _ERRORS:
        return
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "w") as f:
        for r in _ERRORS:
            f.write(json.dumps(r) + "\n")
