"""ctypes binding of libmlxgptq_hip.so (the C ABI in include/mlx_gptq_amd.h).

Only plain pointers, sizes and codes cross the boundary. Tensors must already
live on a HIP device; the helpers here stage host tensors through the device
(never computing on the host) and raise if no HIP device or no built library
is present -- there is deliberately no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import numpy as np
import torch

LIB_PATH = Path(__file__).resolve().parent / "libmlxgptq_hip.so"

OK = 0
ERR_VALUE = -1
ERR_SHAPE = -2
ERR_NOT_PD = -3
ERR_HIP = -4
ERR_WORKSPACE = -5

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

MODE_AFFINE = 0
MODE_MXFP4 = 1
MODE_MXFP8 = 2

CLIP_MINMAX = 0
CLIP_MSE = 1

_VP = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_F32 = ctypes.c_float
_F64 = ctypes.c_double
_SZ = ctypes.c_size_t

# name -> argtypes (every entry point returns int status unless listed in _RESTYPES)
SIGNATURES: dict[str, list] = {
    "mgq_version": [],
    "mgq_last_error": [],
    # grid.py
    "mgq_choose_mxfp_scale": [_VP, _I64, _I64, _INT, _VP, _VP, _VP],
    "mgq_quantize_mxfp_with_scale": [_VP, _VP, _I64, _I64, _INT, _VP, _VP, _VP],
    "mgq_dequantize_mxfp": [_VP, _VP, _I64, _INT, _VP, _VP],
    "mgq_rtn_quantize_mxfp": [_VP, _INT, _I64, _I64, _INT, _VP, _VP, _VP, _VP],
    "mgq_dequantize_affine": [_VP, _VP, _VP, _INT, _I64, _I64, _VP, _VP],
    "mgq_range_audit": [_VP, _INT, _VP, _VP, _VP, _INT, _INT, _I64, _I64, _I64, _VP, _VP],
    "mgq_choose_qparams": [_VP, _I64, _I64, _INT, _INT, _INT, _INT, _F64, _VP, _VP, _VP, _VP, _VP],
    "mgq_quantize_with_params": [_VP, _VP, _VP, _I64, _I64, _INT, _VP, _VP, _VP],
    "mgq_rtn_quantize_affine": [_VP, _INT, _I64, _I64, _INT, _INT, _INT, _INT, _VP, _VP, _VP, _VP, _VP],
    # packing.py / artifacts.py
    "mgq_pack_q": [_VP, _I64, _I64, _INT, _VP, _VP],
    "mgq_unpack_q": [_VP, _I64, _I64, _INT, _I64, _VP, _VP],
    "mgq_pack_nibbles": [_VP, _I64, _I64, _VP, _VP],
    "mgq_unpack_nibbles": [_VP, _I64, _I64, _VP, _VP],
    # capture.py Hessians
    "mgq_hessian_plan": [_I64, _I64, _VP, _I64, _VP, _I64, _VP, _VP],
    "mgq_hessian": [_VP, _I64, _I64, _I64, _VP, _VP, _VP, _INT, _VP, _I64, _VP],
    # gptq.py solver
    "mgq_prepare_hinv_blocks": [_VP, _I64, _I64, _I64, _F32, _INT, _VP, _VP, _VP],
    "mgq_gptq_mxfp_workspace_size": [_I64, _I64, _I64],
    "mgq_gptq_mxfp": [_VP, _INT, _I64, _I64, _I64, _VP, _INT, _INT, _F32, _INT, _VP, _INT,
                      _VP, _VP, _VP, _VP, _VP, _VP, _I64, _VP],
    "mgq_noalloc_scratch_bytes": [],
    "mgq_gptq_mxfp_noalloc": [_VP, _INT, _I64, _I64, _I64, _VP, _INT, _INT, _F32, _INT, _VP, _INT,
                              _VP, _VP, _VP, _VP, _VP, _VP],
    "mgq_gptq_mxfp_prepare": [_VP, _I64, _I64, _I64, _F32, _INT, _VP, _VP, _I64, _VP],
    "mgq_gptq_mxfp_solve": [_VP, _INT, _I64, _I64, _I64, _INT, _INT, _VP, _INT, _VP, _VP, _VP,
                            _VP, _VP, _I64, _VP],
    "mgq_rel_err": [_VP, _VP, _INT, _I64, _I64, _VP, _I64, _VP, _VP],
    "mgq_gptq_mxfp_solve_packed": [_VP, _INT, _I64, _I64, _I64, _INT, _INT, _VP, _INT, _VP, _VP,
                                   _VP, _VP, _VP, _VP, _I64, _VP],
    "mgq_hinv_full_workspace_size": [_I64, _I64],
    "mgq_hinv_full_pass": [_VP, _I64, _I64, _VP, _VP, _VP, _VP, _VP, _I64, _VP],
    "mgq_dead_fix": [_VP, _I64, _I64, _I64, _VP, _VP],
    "mgq_gptq_affine_block": [_VP, _VP, _I64, _I64, _I64, _I64, _I64, _INT, _INT, _INT, _INT,
                              _INT, _F64, _VP, _VP, _VP, _VP, _VP],
}

_RESTYPES = {
    "mgq_last_error": ctypes.c_char_p,
    "mgq_gptq_mxfp_workspace_size": ctypes.c_int64,
    "mgq_noalloc_scratch_bytes": ctypes.c_int64,
    "mgq_hinv_full_workspace_size": ctypes.c_int64,
}

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load the HIP library (once). Raises ImportError if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with "
                    "`python mlx-gptq-mxfp_amd/build.py` (hipcc, gfx950)"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, argtypes in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.argtypes = argtypes
                fn.restype = _RESTYPES.get(name, ctypes.c_int)
            _lib = lib
    return _lib


def last_error() -> str:
    msg = load().mgq_last_error()
    return msg.decode() if msg else ""


def check(rc: int, what: str) -> None:
    if rc == OK:
        return
    msg = last_error() or what
    if rc == ERR_VALUE:
        raise ValueError(msg)
    if rc == ERR_SHAPE:
        raise AssertionError(msg)
    raise RuntimeError(f"{what}: {msg} (status {rc})")


def call(name: str, *args) -> None:
    fn = getattr(load(), name)
    check(fn(*args), name)


# --------------------------------------------------------------------------
# tensor helpers
# --------------------------------------------------------------------------

_DTYPE_CODES = {torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dt]
    except KeyError:
        raise ValueError(f"unsupported dtype {dt} (float32, bfloat16 or float16)") from None


def mode_code(mode: str) -> int:
    if mode == "mxfp4":
        return MODE_MXFP4
    if mode == "mxfp8":
        return MODE_MXFP8
    if mode == "affine":
        return MODE_AFFINE
    raise ValueError(f"unsupported quantization mode: {mode}")


def device_for(*tensors: torch.Tensor) -> torch.device:
    """The HIP device to compute on: the first tensor already on one, else the
    current device. Raises if this process has no HIP device."""
    for t in tensors:
        if isinstance(t, torch.Tensor) and t.is_cuda:
            return t.device
    if not torch.cuda.is_available():
        raise RuntimeError(
            "mlx_gptq (MI355X build) computes on HIP devices only and none is visible; "
            "there is no CPU fallback"
        )
    return torch.device("cuda", torch.cuda.current_device())


def on_device(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    """Contiguous copy/view of ``t`` on ``device``."""
    if t.device != device:
        t = t.to(device, non_blocking=False)
    return t.contiguous()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def numel_groups(shape: tuple[int, ...]) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n


def as_uint8_tensor(q) -> tuple[torch.Tensor, bool]:
    """Accept numpy or torch uint8; report whether the input was numpy."""
    if isinstance(q, np.ndarray):
        return torch.from_numpy(np.ascontiguousarray(q)), True
    return q, False


def library_path() -> str:
    return os.fspath(LIB_PATH)
