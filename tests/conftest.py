"""Test configuration: import paths and the `gpu` marker.

decode-kernel_amd/ is put on sys.path the way the reference puts src/ there
(`PYTHONPATH=src`), so tests import `attention`, `layout` and `dk_lib` directly; the
repository root is on the path for `oracle`.
"""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT / "decode-kernel_amd", ROOT, Path(__file__).resolve().parent):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")
