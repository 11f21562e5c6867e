"""Calibration-row stash and Hessian accumulation on MI355X.

``Stash`` keeps the reference's interface (mlx_gptq/capture.py:33-79: add,
add_sampled, nbytes, hessian, clear) and its numerics: captured rows are
rounded to bf16 (capture.py:49) and H = sum of x^T x in fp32. The product
differs in where rows live -- they stay on the device they were captured on
(HBM is large enough for a layer's calibration set) -- and in how H is
formed: one bf16-MFMA SYRK launch (csrc/hessian.hip) instead of chunked fp32
``addmm``.

``grouped_hessian`` is the batched form used for routed experts: every
expert's H from one hidden-state matrix plus a per-expert token list, with
the gather fused into the MFMA tile loads.
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import numpy as np
import torch

from . import _native as nat


def _as_offsets(offsets) -> np.ndarray:
    if isinstance(offsets, torch.Tensor):
        offsets = offsets.detach().to("cpu", torch.int64).numpy()
    off = np.ascontiguousarray(np.asarray(offsets, dtype=np.int64))
    if off.ndim != 1 or off.size < 2:
        raise ValueError("offsets must be a 1-D sequence of n_groups + 1 entries")
    if np.any(np.diff(off) < 0) or off[0] < 0:
        raise ValueError("offsets must be non-negative and non-decreasing")
    return off


def grouped_hessian(
    X: torch.Tensor,
    offsets: Sequence[int] | np.ndarray | torch.Tensor,
    row_index: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    accumulate: bool = False,
    target_items: int = 0,
    validate: bool = True,
) -> torch.Tensor:
    """H[g] (+)= X_g^T X_g for every group g, fp32 [G, C, C].

    X: bf16 [N, C] on a HIP device (row-contiguous). Group g uses the token
    list entries offsets[g]:offsets[g+1]; entry t selects row
    ``row_index[t]`` of X (or row t when ``row_index`` is None).
    ``validate`` checks the gather indices first (one device reduction and a
    host sync); the kernel never reads outside X either way.
    """
    if X.dtype != torch.bfloat16:
        raise TypeError(f"grouped_hessian expects bfloat16 rows (got {X.dtype})")
    if X.dim() != 2 or X.stride(1) != 1:
        raise ValueError("X must be a row-contiguous [N, C] matrix")
    dev = nat.device_for(X)
    if not X.is_cuda:
        X = X.to(dev)
    off = _as_offsets(offsets)
    G = off.size - 1
    C = int(X.shape[1])
    if row_index is not None:
        row_index = nat.on_device(row_index.to(torch.int32), dev)
        if int(off[-1]) > row_index.numel():
            raise ValueError("offsets exceed the token list")
        if validate and row_index.numel():
            lo, hi = torch.aminmax(row_index[: int(off[-1])])
            if int(lo) < 0 or int(hi) >= X.shape[0]:
                raise IndexError(f"row_index outside [0, {X.shape[0]})")
    elif int(off[-1]) > X.shape[0]:
        raise ValueError("offsets exceed the rows of X")
    if out is None:
        out = torch.empty(G, C, C, dtype=torch.float32, device=dev)
        accumulate = False
    elif out.shape != (G, C, C) or out.dtype != torch.float32 or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous float32 [{G}, {C}, {C}] tensor")
    lib = nat.load()
    plan_bytes = ctypes.c_int64(0)
    ws_bytes = ctypes.c_int64(0)
    nat.check(
        lib.mgq_hessian_plan(C, G, off.ctypes.data, int(target_items), None, 0,
                             ctypes.byref(plan_bytes), ctypes.byref(ws_bytes)),
        "mgq_hessian_plan",
    )
    plan = torch.empty(plan_bytes.value, dtype=torch.uint8, pin_memory=True)
    nat.check(
        lib.mgq_hessian_plan(C, G, off.ctypes.data, int(target_items), plan.data_ptr(),
                             plan_bytes.value, None, None),
        "mgq_hessian_plan",
    )
    ws = torch.empty(ws_bytes.value, dtype=torch.uint8, device=dev)
    ws[: plan_bytes.value].copy_(plan, non_blocking=True)
    nat.call(
        "mgq_hessian", X.data_ptr(), int(X.shape[0]), X.stride(0), C,
        None if row_index is None else row_index.data_ptr(), plan.data_ptr(), out.data_ptr(),
        1 if accumulate else 0, ws.data_ptr(), ws_bytes.value, nat.stream_of(dev),
    )
    return out


def hessian_xtx(X: torch.Tensor, out: torch.Tensor | None = None, accumulate: bool = False) -> torch.Tensor:
    """Dense H = X^T X (fp32 [C, C]) of bf16 rows X [N, C]."""
    H = grouped_hessian(X, [0, int(X.shape[0])], None,
                        None if out is None else out.unsqueeze(0), accumulate)
    return H[0]


class Stash:
    """Captured input rows for one logical weight matrix (capture.py:33-79)."""

    def __init__(self, name: str, in_features: int):
        self.name = name
        self.in_features = in_features
        self.chunks: list[torch.Tensor] = []
        self.tokens = 0

    def add(self, x: torch.Tensor):
        rows = x.detach().reshape(-1, x.shape[-1])
        if rows.shape[-1] != self.in_features:
            raise RuntimeError(
                f"stash {self.name}: got rows of dim {rows.shape[-1]}, "
                f"expected {self.in_features}"
            )
        # bf16 rounding as capture.py:49; rows stay on their device.
        self.chunks.append(rows.to(torch.bfloat16).contiguous())
        self.tokens += rows.shape[0]

    def add_sampled(self, x: torch.Tensor, max_rows: int):
        """Deterministic, evenly spaced sample of rows (capture.py:52-63)."""
        rows = x.detach().reshape(-1, x.shape[-1])
        if rows.shape[0] > max_rows:
            idx = torch.linspace(0, rows.shape[0] - 1, steps=max_rows, device=rows.device).long()
            rows = rows.index_select(0, idx)
        self.add(rows)

    def nbytes(self) -> int:
        return sum(c.numel() * 2 for c in self.chunks)

    @torch.no_grad()
    def hessian(self, device, chunk_rows: int = 65536) -> torch.Tensor:
        """H = X^T X in fp32 on `device` (capture.py:68-76)."""
        dev = torch.device(device)
        if dev.type != "cuda":
            raise RuntimeError(
                "mlx_gptq (MI355X build) accumulates Hessians on HIP devices only "
                f"(got device {dev})"
            )
        C = self.in_features
        H = torch.zeros(C, C, dtype=torch.float32, device=dev)
        first = True
        for c in self.chunks:
            for i in range(0, c.shape[0], chunk_rows):
                x = c[i : i + chunk_rows]
                if x.device != dev:
                    x = x.to(dev, non_blocking=True)
                if x.shape[0] == 0:
                    continue
                hessian_xtx(x, out=H, accumulate=not first)
                first = False
        return H

    def clear(self):
        self.chunks.clear()
