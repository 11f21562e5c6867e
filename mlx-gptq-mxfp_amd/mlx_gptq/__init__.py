"""MI355X-native GPTQ calibration solver behind the mlx_gptq solver API.

Modules mirror the reference package's solver path (gptq.py, grid.py,
packing.py, artifacts.py, capture.py, pack.py, validate_artifacts.py); all
arithmetic runs in hand-written gfx950 HIP kernels (libmlxgptq_hip.so, C ABI
in include/mlx_gptq_amd.h).

Drop-in with a reference checkout: set ``MLX_GPTQ_REFERENCE`` to the
checkout (its root or its ``mlx_gptq`` directory). That directory is then
appended to this package's ``__path__``, so the modules this build does not
provide (``calibrate``, ``sequential``, ``data``, ``flint_torch``, ...)
import from the checkout, while every module present here -- the solver,
capture, artifacts and Stage-B modules -- shadows the reference's.
"""

import os as _os

__version__ = "0.2.0"


def _extend_path() -> None:
    ref = _os.environ.get("MLX_GPTQ_REFERENCE")
    if not ref:
        return
    sub = _os.path.join(ref, "mlx_gptq")
    pkg_dir = sub if _os.path.isdir(sub) else ref
    if not _os.path.isfile(_os.path.join(pkg_dir, "__init__.py")):
        raise ImportError(f"MLX_GPTQ_REFERENCE={ref!r} holds no mlx_gptq package")
    pkg_dir = _os.path.abspath(pkg_dir)
    if pkg_dir not in [_os.path.abspath(p) for p in __path__]:
        __path__.append(pkg_dir)


_extend_path()
