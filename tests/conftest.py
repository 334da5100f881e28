import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "llm-kv260_amd"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs through the C ABI")
    config.addinivalue_line("markers", "slow: CPU test that takes more than a few seconds")


@pytest.fixture(scope="session")
def gpu():
    """The HIP library, loaded, with device 0 current. Fails (not skips) when
    the extension is missing: a GPU test must never pass on a fallback."""
    import torch  # noqa: F401  (loads torch's HIP runtime first; the library then shares it)
    import kv260gemv
    if not torch.cuda.is_available():
        pytest.fail("GPU test collected but no GPU is visible")
    kv260gemv.require_device()
    return kv260gemv
