import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "verified-metal-kernels_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "tests"), os.path.join(PKG, "kernels")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libvmk.so")
