import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

import __graft_entry__  # noqa: E402

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def pkg():
    """The plugin package (comfyui-featherops_amd/) imported as `featherops_amd`."""
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def hk(pkg):
    import importlib

    return importlib.import_module("featherops_amd.kernel.hip.hip_kernel")


@pytest.fixture(scope="session")
def quant(pkg):
    import importlib

    return importlib.import_module("featherops_amd.comfy_feather.quant")


@pytest.fixture(scope="session")
def cuda():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test ran without a GPU")
    return torch.device("cuda:0")
