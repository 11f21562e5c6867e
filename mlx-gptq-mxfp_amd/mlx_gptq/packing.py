"""MLX uint32 bit-packing of quantized codes on MI355X (packing.py API).

Layout (reference mlx_gptq/packing.py:1-12): 32/bits consecutive codes per
uint32 word, first code in the least-significant bits; 2, 4 and 8 bits. The
packing runs in csrc/pack.hip. numpy inputs are staged through the current HIP
device and come back as numpy, so Stage-B style callers keep working.
"""

from __future__ import annotations

import numpy as np
import torch

from . import _native as nat

PACKABLE_BITS = (2, 4, 8)


def pack_q(q, bits: int):
    """q: uint8 [..., C] (numpy or torch) -> uint32 [..., C*bits/32] (packing.py:15-26)."""
    if bits not in PACKABLE_BITS:
        raise ValueError(f"cannot pack {bits}-bit for MLX (supported: {PACKABLE_BITS})")
    per = 32 // bits
    t, was_np = nat.as_uint8_tensor(q)
    *lead, C = t.shape
    assert C % per == 0, f"last dim {C} not divisible by {per}"
    if t.dtype != torch.uint8:
        t = t.to(torch.uint8)
    dev = nat.device_for(t)
    x = nat.on_device(t, dev)
    rows = nat.numel_groups(tuple(lead))
    words = torch.empty((*lead, C // per), dtype=torch.int32, device=dev)
    if rows and C:
        nat.call("mgq_pack_q", x.data_ptr(), rows, C, bits, words.data_ptr(), nat.stream_of(dev))
    if was_np:
        return words.cpu().numpy().view(np.uint32)
    return words.view(torch.uint32).to(t.device) if hasattr(torch, "uint32") else words.to(t.device)


def pack_mxfp4(q):
    """Pack E2M1 codes into the native MLX MXFP4 uint32 layout (packing.py:29-31)."""
    return pack_q(q, 4)


def unpack_q(words, bits: int, out_cols: int):
    """uint32 words [..., W] -> uint8 codes [..., out_cols] (packing.py:34-39)."""
    was_np = isinstance(words, np.ndarray)
    if was_np:
        t = torch.from_numpy(np.ascontiguousarray(words).view(np.int32))
    else:
        t = words.view(torch.int32) if words.dtype != torch.int32 else words
    *lead, n_words = t.shape
    dev = nat.device_for(t)
    x = nat.on_device(t, dev)
    rows = nat.numel_groups(tuple(lead))
    out_cols = min(int(out_cols), n_words * (32 // bits))
    q = torch.empty((*lead, out_cols), dtype=torch.uint8, device=dev)
    if rows and out_cols:
        nat.call(
            "mgq_unpack_q", x.data_ptr(), rows, n_words, bits, out_cols, q.data_ptr(),
            nat.stream_of(dev),
        )
    if was_np:
        return q.cpu().numpy()
    return q.to(t.device)
