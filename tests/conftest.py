import os
import sys

import pytest

# torch ships its own libamdhip64.so.7 and libqqmoe.so needs that soname too:
# whichever is loaded first serves both.  torch's must be the one (torch
# initialises no device with another build's runtime), so torch is imported
# before any test loads the library.
try:
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "qwenqwen3.js_amd", "tests"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libqqmoe.so")
