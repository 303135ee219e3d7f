import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
for sub in ("turbo-winfare_amd", "oracle", "tests"):
    p = str(ROOT / sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
