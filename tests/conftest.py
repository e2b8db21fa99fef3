import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def engine():
    from aether_nexus_amd.weaver import WeaverEngine
    eng = WeaverEngine()
    yield eng
    eng.close()


@pytest.fixture(scope="session")
def stream():
    import torch
    return torch.cuda.current_stream().cuda_stream
