import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# the repo root (for `oracle`) and the package directory (for `mojodgl`)
for path in (ROOT, os.path.join(ROOT, "mojo-dgl_amd")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmdgl.so)")
