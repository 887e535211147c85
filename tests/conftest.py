import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "mlx-swift-diffrast_amd"), os.path.join(ROOT, "oracle"),
          os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def fixtures():
    """nvdiffrast (CUDA) reference outputs shipped with the reference's tests
    (Tests/MLXDiffRastTests/Fixtures/diffrast_fixtures.safetensors)."""
    from safetensors.numpy import load_file
    return load_file(os.path.join(ROOT, "tests", "golden", "diffrast_fixtures.safetensors"))
