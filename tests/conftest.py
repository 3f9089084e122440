import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "qwen-mlx-runner_amd", ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; fails without one")


@pytest.fixture(scope="session")
def gpu():
    """The default device: GEMV variant "aligned", FP32 metadata mode."""
    import qmr

    g = qmr.Gpu("aligned")
    yield g
    g.close()


@pytest.fixture(scope="session")
def gpus():
    """One device handle per reference GEMV mode (tests/quantized.rs:8-11)."""
    import qmr

    handles = {
        "packed4": qmr.Gpu("packed4"),
        "aligned": qmr.Gpu("aligned"),
        "stream": qmr.Gpu("stream"),
        "reference": qmr.Gpu("aligned", reference=True),
    }
    yield handles
    for g in handles.values():
        g.close()
