import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = Path(__file__).resolve().parent / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libintent_hip.so")


@pytest.fixture(scope="session")
def golden():
    cache = {}

    def load(name):
        if name not in cache:
            with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as data:
                cache[name] = {key: data[key] for key in data.files}
        return cache[name]

    return load


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    from intent_amd.runtime.hip.library import library

    info = library().device_info(0)
    if not info["arch"].startswith("gfx950"):
        pytest.skip(f"device 0 is {info['arch']}, not gfx950")
    return torch.device("cuda", 0)
