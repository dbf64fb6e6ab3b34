import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "data-synth-tpu_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and libq6moe.so")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    from q6moe import _lib

    _lib.load()  # fail loudly if the extension is missing
    return torch.device("cuda", 0)


def pytest_runtest_setup(item):
    if "gpu" in item.keywords:
        print(f"\n[gpu-test] {item.nodeid}", flush=True)
    os.environ.setdefault("PYTHONHASHSEED", "0")
