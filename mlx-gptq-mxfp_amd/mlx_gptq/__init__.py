"""MI355X-native GPTQ calibration solver behind the mlx_gptq solver API.

Modules mirror the reference package's solver path (gptq.py, grid.py,
packing.py, artifacts.py nibble packing, capture.py Hessians); all arithmetic
runs in hand-written gfx950 HIP kernels (libmlxgptq_hip.so, C ABI in
include/mlx_gptq_amd.h).
"""

__version__ = "0.1.0"
