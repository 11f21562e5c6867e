"""Nibble packing for calibration artifacts (artifacts.py:30-39 API) on MI355X.

4-bit codes are stored two per byte, low nibble first. The on-disk artifact
store itself (manifest + safetensors) is not part of the solver path.
"""

from __future__ import annotations

import torch

from . import _native as nat


def pack_nibbles(q: torch.Tensor) -> torch.Tensor:
    """uint8 [..., C] -> uint8 [..., C/2] with byte = q[2k] | q[2k+1] << 4 (artifacts.py:30-32)."""
    assert q.dtype == torch.uint8 and q.shape[-1] % 2 == 0
    dev = nat.device_for(q)
    x = nat.on_device(q, dev)
    *lead, C = q.shape
    rows = nat.numel_groups(tuple(lead))
    out = torch.empty((*lead, C // 2), dtype=torch.uint8, device=dev)
    if rows and C:
        nat.call("mgq_pack_nibbles", x.data_ptr(), rows, C, out.data_ptr(), nat.stream_of(dev))
    return out.to(q.device)


def unpack_nibbles(p: torch.Tensor) -> torch.Tensor:
    """uint8 [..., P] -> uint8 [..., 2P], low nibble first (artifacts.py:35-39)."""
    dev = nat.device_for(p)
    x = nat.on_device(p.to(torch.uint8), dev)
    *lead, P = p.shape
    rows = nat.numel_groups(tuple(lead))
    out = torch.empty((*lead, 2 * P), dtype=torch.uint8, device=dev)
    if rows and P:
        nat.call("mgq_unpack_nibbles", x.data_ptr(), rows, P, out.data_ptr(), nat.stream_of(dev))
    return out.to(p.device)
