import os
import sys

import pytest

# PyTorch-ROCm ships its own HIP runtime.  When libgtmoe (linked against the
# system's) starts HIP first in a process, torch's runtime then finds no
# device; with torch loaded first, libgtmoe binds to the runtime already in
# the process and both see the GPU.  So torch, when installed, is imported
# before any test module loads the library.
try:
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")
