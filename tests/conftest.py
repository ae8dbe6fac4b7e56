import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP kernels")
    # The oracle's C library is built here, before anything in this process touches a GPU; the
    # oracle's loader itself never builds (tests may hold a GPU context by then).
    if not (ROOT / "oracle" / "liboracle.so").exists():
        import subprocess

        subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def cuda():
    if not gpu_available():
        pytest.skip("no GPU visible")
    import torch

    return torch.device("cuda", 0)
