"""pytest setup: import paths and the `gpu` marker.

The product package lives in ``mlx-gptq-mxfp_amd/mlx_gptq`` (a directory name
that is not a Python identifier), so it is put on sys.path here; ``oracle``
is imported from the repository root.
"""

from __future__ import annotations

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "mlx-gptq-mxfp_amd")
for p in (PKG, ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X) and the built library")
