"""Restatement of the reference Hessian accumulation (test oracle only).

capture.py:42-50 stores captured rows as CPU bf16; capture.py:68-76 builds
H = sum over 65536-row chunks of x^T x with fp32 ``addmm_`` on a zero H.
"""

from __future__ import annotations

import torch


def stash_hessian(chunks, in_features: int, chunk_rows: int = 65536, device="cpu") -> torch.Tensor:
    """capture.py:68-76 over a list of bf16 [n_i, C] chunks."""
    H = torch.zeros(in_features, in_features, dtype=torch.float32, device=device)
    for c in chunks:
        for i in range(0, c.shape[0], chunk_rows):
            x = c[i : i + chunk_rows].to(device, torch.float32)
            H.addmm_(x.T, x)
    return H


def hessian_fp64(X_bf16: torch.Tensor) -> torch.Tensor:
    """Exact-ish reference: X^T X of the same bf16 rows in float64."""
    x = X_bf16.to(torch.float64)
    return x.T @ x


def rel_frobenius(H: torch.Tensor, ref: torch.Tensor) -> float:
    ref = ref.to(torch.float64)
    return float((H.to(torch.float64) - ref).norm() / ref.norm().clamp_min(1e-300))
