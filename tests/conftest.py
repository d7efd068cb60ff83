import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "tests", ROOT / "tests" / "golden"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def gpu():
    """A dedicated HIP stream on cuda:0 (the library rejects the null stream)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from raftinfer_amd import _lib
    _lib.load()
    torch.cuda.init()
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        yield stream
    torch.cuda.synchronize()
