"""Affine (MLX scale/bias) GPTQ path: full-matrix damped Cholesky-inverse and
the lazy-block column loop (gptq.py:229-272). See csrc/gptq_affine.hip."""

from __future__ import annotations

import torch

from . import _native as nat


def rel_err(W_dq: torch.Tensor, W_orig: torch.Tensor) -> torch.Tensor:
    """||W_dq - W_orig||_F / max(||W_orig||_F, 1e-12) per batch item (gptq.py:300-302)."""
    W0 = W_orig.to(W_dq.device).float()
    num = (W_dq - W0).pow(2).sum(dim=(1, 2)).sqrt()
    den = W0.pow(2).sum(dim=(1, 2)).sqrt().clamp(min=1e-12)
    return num / den


def prepare_hinv_full(H: torch.Tensor, damp: float, max_attempts: int):
    raise NotImplementedError("full-matrix Cholesky inverse: not built yet")


def gptq_quantize_affine(W, H, bits, group_size, damp, clip, storage_dtype, block_size):
    raise NotImplementedError("affine GPTQ path: not built yet")
