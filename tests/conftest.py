import os
import pathlib
import sys

import pytest

REPO = pathlib.Path(__file__).resolve().parent.parent
for p in (REPO, REPO / "flash-hog_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def cuda_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


def pytest_report_header(config):
    return f"flash-hog tests, repo {REPO}, FLASH_HOG_HIP_LIB={os.environ.get('FLASH_HOG_HIP_LIB', '<in-tree>')}"
