"""numpy / torch-CPU restatement of the reference packers (test oracle only).

packing.py:15-39 (numpy uint32, LSB-first) and artifacts.py:30-39 (nibbles).
"""

from __future__ import annotations

import numpy as np
import torch


def pack_q(q: np.ndarray, bits: int) -> np.ndarray:
    """packing.py:15-26."""
    if bits not in (2, 4, 8):
        raise ValueError(f"cannot pack {bits}-bit for MLX (supported: (2, 4, 8))")
    per = 32 // bits
    *lead, C = q.shape
    assert C % per == 0, f"last dim {C} not divisible by {per}"
    grouped = q.reshape(*lead, C // per, per).astype(np.uint32)
    out = np.zeros((*lead, C // per), dtype=np.uint32)
    for i in range(per):
        out |= grouped[..., i] << np.uint32(bits * i)
    return out


def unpack_q(words: np.ndarray, bits: int, out_cols: int) -> np.ndarray:
    """packing.py:34-39."""
    per = 32 // bits
    mask = (1 << bits) - 1
    parts = np.stack([(words >> (bits * i)) & mask for i in range(per)], axis=-1)
    return parts.reshape(*words.shape[:-1], words.shape[-1] * per)[..., :out_cols].astype(np.uint8)


def pack_nibbles(q: torch.Tensor) -> torch.Tensor:
    """artifacts.py:30-32."""
    assert q.dtype == torch.uint8 and q.shape[-1] % 2 == 0
    return q[..., 0::2] | (q[..., 1::2] << 4)


def unpack_nibbles(p: torch.Tensor) -> torch.Tensor:
    """artifacts.py:35-39."""
    return torch.stack([p & 0xF, p >> 4], dim=-1).reshape(*p.shape[:-1], p.shape[-1] * 2)
