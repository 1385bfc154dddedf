import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (runs through the C ABI on the device)")
    # tuning decisions of a test run persist in a table of its own, not the user's
    if "BORCH_AMD_PLAN_CACHE" not in os.environ:
        import tempfile
        os.environ["BORCH_AMD_PLAN_CACHE"] = os.path.join(tempfile.mkdtemp(prefix="bq-plans-"), "plans.json")


@pytest.fixture(scope="session")
def dev():
    """The GPU, or a failure: a gpu-marked test never passes on a CPU fallback."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test without a visible GPU")
    import borch_amd._lib as L
    L.require_device(torch.device("cuda:0"))
    return torch.device("cuda:0")
