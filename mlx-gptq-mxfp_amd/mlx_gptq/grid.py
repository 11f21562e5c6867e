"""MLX quantization grids (affine, MXFP4 E2M1+E8M0, MXFP8 E4M3+E8M0) on MI355X.

Same names, signatures, shapes and error types as the reference module
mlx_gptq/grid.py; every element-wise computation runs in the HIP kernels of
libmlxgptq_hip.so (csrc/grid.hip) and reproduces the reference's fp32
arithmetic bit for bit:

  - MLX affine: w = q*scale + bias, q in [0, 2**bits-1], scale/bias rounded to
    the storage dtype before q is computed (grid.py:1-13, 167-221);
  - MXFP: one E8M0 power-of-two scale per 32 consecutive inputs, chosen as
    round-half-even(log2(max|w| / fmax)) (grid.py:61-79), E2M1 via the
    saturating RNE thresholds (grid.py:82-105), E4M3 via clamp(+-448) and an
    RNE cast (grid.py:108-124).

Host tensors are staged through the current HIP device and results returned
on the caller's device; there is no CPU compute path.
"""

from __future__ import annotations

import torch

from . import _native as nat

SUPPORTED_BITS = (2, 4, 8)
SUPPORTED_MODES = ("affine", "mxfp4", "mxfp8")
MX_GROUP_SIZE = 32

_E2M1_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)


def mode_defaults(mode: str) -> tuple[int, int]:
    """(group_size, bits) defaults per mode (grid.py:43-50)."""
    if mode == "mxfp4":
        return MX_GROUP_SIZE, 4
    if mode == "mxfp8":
        return MX_GROUP_SIZE, 8
    if mode == "affine":
        return 64, 4
    raise ValueError(f"unsupported quantization mode: {mode}")


def _mxfp_max(mode: str) -> float:
    """Largest finite grid value (grid.py:53-58)."""
    if mode == "mxfp4":
        return 6.0
    if mode == "mxfp8":
        return 448.0
    raise ValueError(f"not a microscaling mode: {mode}")


def _storage_code(dt: torch.dtype) -> int:
    return nat.dtype_code(dt)


def _clip_code(method: str) -> int:
    """grid.py:187-192: "minmax" keeps the full range; any other method is
    the MSE range-shrink search."""
    return nat.CLIP_MINMAX if method == "minmax" else nat.CLIP_MSE


def _require_f32(t: torch.Tensor, fn: str) -> None:
    if t.dtype != torch.float32:
        raise TypeError(f"{fn}: expects float32 values (got {t.dtype}); call .float() first")


def choose_mxfp_scale(w: torch.Tensor, mode: str):
    """E8M0 scale per group along the last axis (grid.py:61-79).

    Returns (scale_bytes uint8 [...], scales float32 [...]).
    """
    _mxfp_max(mode)
    _require_f32(w, "choose_mxfp_scale")
    dev = nat.device_for(w)
    x = nat.on_device(w, dev)
    lead = tuple(w.shape[:-1])
    k = int(w.shape[-1])
    if k == 0:
        raise RuntimeError("choose_mxfp_scale: amax over an empty dimension")
    n = nat.numel_groups(lead)
    b = torch.empty(lead, dtype=torch.uint8, device=dev)
    s = torch.empty(lead, dtype=torch.float32, device=dev)
    nat.call(
        "mgq_choose_mxfp_scale", x.data_ptr(), n, k, nat.mode_code(mode), b.data_ptr(),
        s.data_ptr(), nat.stream_of(dev),
    )
    return b.to(w.device), s.to(w.device)


def _e2m1_codes(x: torch.Tensor) -> torch.Tensor:
    """E2M1 codes of already-normalized values (grid.py:82-105)."""
    _require_f32(x, "_e2m1_codes")
    ones = torch.ones(x.shape[:-1] if x.dim() else (), dtype=torch.float32, device=x.device)
    if x.dim() == 0:
        q, _ = quantize_mxfp_with_scale(x.reshape(1, 1), ones.reshape(1), "mxfp4")
        return q.reshape(())
    q, _ = quantize_mxfp_with_scale(x, ones, "mxfp4")
    return q


def quantize_mxfp_with_scale(w: torch.Tensor, scales: torch.Tensor, mode: str):
    """Project onto the MXFP grid with fixed per-group scales (grid.py:108-124).

    w: [..., k] float32, scales: [...] -> (q uint8 [..., k], dq float32 [..., k]).
    """
    if mode not in ("mxfp4", "mxfp8"):
        raise ValueError(f"not a microscaling mode: {mode}")
    _require_f32(w, "quantize_mxfp_with_scale")
    dev = nat.device_for(w, scales)
    x = nat.on_device(w, dev)
    lead = tuple(w.shape[:-1])
    sc = nat.on_device(scales.to(torch.float32).expand(lead), dev)
    k = int(w.shape[-1])
    n = nat.numel_groups(lead)
    q = torch.empty(w.shape, dtype=torch.uint8, device=dev)
    dq = torch.empty(w.shape, dtype=torch.float32, device=dev)
    if k > 0 and n > 0:
        nat.call(
            "mgq_quantize_mxfp_with_scale", x.data_ptr(), sc.data_ptr(), n, k,
            nat.mode_code(mode), q.data_ptr(), dq.data_ptr(), nat.stream_of(dev),
        )
    return q.to(w.device), dq.to(w.device)


def dequantize_mxfp(q: torch.Tensor, scale_bytes: torch.Tensor, mode: str):
    """Codes + E8M0 bytes -> float32 [..., C/32, 32] (grid.py:127-139)."""
    if mode not in ("mxfp4", "mxfp8"):
        raise ValueError(f"not a microscaling mode: {mode}")
    C = int(q.shape[-1])
    if C % MX_GROUP_SIZE:
        raise RuntimeError(f"shape of q {tuple(q.shape)} is not a multiple of {MX_GROUP_SIZE}")
    dev = nat.device_for(q, scale_bytes)
    qq = nat.on_device(q.to(torch.uint8), dev)
    out_shape = (*q.shape[:-1], C // MX_GROUP_SIZE, MX_GROUP_SIZE)
    n_groups = nat.numel_groups(out_shape[:-1])
    sb = nat.on_device(scale_bytes.to(torch.uint8).reshape(out_shape[:-1]), dev)
    out = torch.empty(out_shape, dtype=torch.float32, device=dev)
    if n_groups:
        nat.call(
            "mgq_dequantize_mxfp", qq.data_ptr(), sb.data_ptr(), n_groups, nat.mode_code(mode),
            out.data_ptr(), nat.stream_of(dev),
        )
    return out.to(q.device)


@torch.no_grad()
def rtn_quantize_mxfp(W: torch.Tensor, mode: str):
    """Native MXFP round-to-nearest (grid.py:142-151).

    Returns (q uint8 [..., R, C], scale_bytes uint8 [..., R, C/32], None, dq f32 [..., R, C]).
    """
    *lead, rows, columns = W.shape
    if columns % MX_GROUP_SIZE:
        raise ValueError(f"columns {columns} not divisible by {MX_GROUP_SIZE}")
    if mode not in ("mxfp4", "mxfp8"):
        raise ValueError(f"not a microscaling mode: {mode}")
    dev = nat.device_for(W)
    src = W if W.dtype in (torch.float32, torch.bfloat16, torch.float16) else W.float()
    x = nat.on_device(src, dev)
    R = nat.numel_groups((*lead, rows))
    q = torch.empty((*lead, rows, columns), dtype=torch.uint8, device=dev)
    sb = torch.empty((*lead, rows, columns // MX_GROUP_SIZE), dtype=torch.uint8, device=dev)
    dq = torch.empty((*lead, rows, columns), dtype=torch.float32, device=dev)
    if R and columns:
        nat.call(
            "mgq_rtn_quantize_mxfp", x.data_ptr(), nat.dtype_code(x.dtype), R, columns,
            nat.mode_code(mode), q.data_ptr(), sb.data_ptr(), dq.data_ptr(), nat.stream_of(dev),
        )
    return q.to(W.device), sb.to(W.device), None, dq.to(W.device)


def dequantize_artifact(q: torch.Tensor, scales: torch.Tensor, biases, mode: str, group_size: int):
    """Dequantize one stored artifact (grid.py:154-164)."""
    if mode == "affine":
        dev = nat.device_for(q, scales)
        qq = nat.on_device(q.to(torch.uint8), dev)
        G = int(group_size)
        if q.shape[-1] % G:
            raise RuntimeError(f"shape of q {tuple(q.shape)} is not a multiple of {G}")
        n_groups = q.numel() // G
        if scales.dtype != biases.dtype or scales.dtype not in (
            torch.float32, torch.bfloat16, torch.float16,
        ):
            scales, biases = scales.float(), biases.float()
        s = nat.on_device(scales.reshape(-1), dev)
        b = nat.on_device(biases.reshape(-1), dev)
        out = torch.empty(q.shape, dtype=torch.float32, device=dev)
        if n_groups:
            nat.call(
                "mgq_dequantize_affine", qq.data_ptr(), s.data_ptr(), b.data_ptr(),
                nat.dtype_code(s.dtype), n_groups, G, out.data_ptr(), nat.stream_of(dev),
            )
        return out.to(q.device)
    if group_size != MX_GROUP_SIZE:
        raise ValueError(f"{mode} requires group size {MX_GROUP_SIZE}")
    return dequantize_mxfp(q, scales, mode).reshape(q.shape)


def choose_qparams(
    w: torch.Tensor,
    bits: int,
    method: str = "mse",
    storage_dtype: torch.dtype = torch.bfloat16,
    grid_steps: int = 20,
    max_shrink: float = 0.2,
):
    """Per-group affine scale/bias with MSE range-shrink search (grid.py:167-212).

    Returns (scales_stored, biases_stored, scales_f32, biases_f32), shape [...].
    """
    _require_f32(w, "choose_qparams")
    dev = nat.device_for(w)
    x = nat.on_device(w, dev)
    lead = tuple(w.shape[:-1])
    n = nat.numel_groups(lead)
    k = int(w.shape[-1])
    s_st = torch.empty(lead, dtype=storage_dtype, device=dev)
    b_st = torch.empty(lead, dtype=storage_dtype, device=dev)
    s32 = torch.empty(lead, dtype=torch.float32, device=dev)
    b32 = torch.empty(lead, dtype=torch.float32, device=dev)
    if n:
        nat.call(
            "mgq_choose_qparams", x.data_ptr(), n, k, int(bits),
            _clip_code(method), _storage_code(storage_dtype),
            int(grid_steps), float(max_shrink), s_st.data_ptr(), b_st.data_ptr(), s32.data_ptr(),
            b32.data_ptr(), nat.stream_of(dev),
        )
    to = w.device
    return s_st.to(to), b_st.to(to), s32.to(to), b32.to(to)


def quantize_with_params(w, s32, b32, bits):
    """Quantize [..., G] values with f32 params (grid.py:215-221) -> (q f32, dq f32)."""
    _require_f32(w, "quantize_with_params")
    dev = nat.device_for(w, s32, b32)
    x = nat.on_device(w, dev)
    lead = tuple(w.shape[:-1])
    s = nat.on_device(s32.to(torch.float32).expand(lead), dev)
    b = nat.on_device(b32.to(torch.float32).expand(lead), dev)
    n = nat.numel_groups(lead)
    k = int(w.shape[-1])
    q = torch.empty(w.shape, dtype=torch.float32, device=dev)
    dq = torch.empty(w.shape, dtype=torch.float32, device=dev)
    if n and k:
        nat.call(
            "mgq_quantize_with_params", x.data_ptr(), s.data_ptr(), b.data_ptr(), n, k, int(bits),
            q.data_ptr(), dq.data_ptr(), nat.stream_of(dev),
        )
    return q.to(w.device), dq.to(w.device)


@torch.no_grad()
def rtn_quantize(
    W: torch.Tensor,
    bits: int,
    group_size: int,
    method: str = "mse",
    storage_dtype: torch.dtype = torch.bfloat16,
):
    """Affine round-to-nearest on the MLX grid (grid.py:224-246).

    Returns (q uint8 [..., R, C], scales, biases [..., R, C/G], W_dq f32).
    """
    *lead, R, C = W.shape
    assert C % group_size == 0, f"cols {C} not divisible by group size {group_size}"
    dev = nat.device_for(W)
    x = nat.on_device(W.float(), dev)
    rows = nat.numel_groups((*lead, R))
    G = int(group_size)
    q = torch.empty((*lead, R, C), dtype=torch.uint8, device=dev)
    s_st = torch.empty((*lead, R, C // G), dtype=storage_dtype, device=dev)
    b_st = torch.empty((*lead, R, C // G), dtype=storage_dtype, device=dev)
    dq = torch.empty((*lead, R, C), dtype=torch.float32, device=dev)
    if rows and C:
        nat.call(
            "mgq_rtn_quantize_affine", x.data_ptr(), nat.DTYPE_F32, rows, C, int(bits), G,
            _clip_code(method), _storage_code(storage_dtype),
            q.data_ptr(), s_st.data_ptr(), b_st.data_ptr(), dq.data_ptr(), nat.stream_of(dev),
        )
    to = W.device
    return q.to(to), s_st.to(to), b_st.to(to), dq.to(to)
