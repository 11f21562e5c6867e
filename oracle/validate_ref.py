"""torch-CPU restatement of the reference's artifact range audit (test
oracle only): validate_artifacts.py:15-55 for one tensor.

Pinned by tests/test_range_audit.py on closed-form cases (a group that
dequantizes exactly to its source: ratio 1/32; codes scaled past the limit:
ratio = the scale factor / 32; an all-zero source group: limit 2^-126; an
E8M0 byte of 255: infinite values), on top of which the random cases
compare it with the GPU.
"""

from __future__ import annotations

import torch

from . import grid_ref

MX_GROUP_SIZE = 32


def _group_max(value: torch.Tensor) -> torch.Tensor:
    """validate_artifacts.py:15-18."""
    rows, columns = value.shape
    return value.reshape(rows, columns // MX_GROUP_SIZE, MX_GROUP_SIZE).abs().amax(dim=-1)


def range_audit(source, q, scales, biases, mode: str, group_size: int) -> dict:
    """validate_artifacts.py:29-55: the stats the report is made of."""
    source = source.float()
    deq = grid_ref.dequantize_artifact(q, scales, biases, mode, group_size)
    smax = _group_max(source)
    amax = _group_max(deq)
    limit = torch.maximum(smax.to(torch.float64) * 32.0, torch.full_like(smax, 2.0**-126))
    ratios = amax.to(torch.float64) / limit
    return {
        "nonfinite": int((~torch.isfinite(deq)).sum()),
        "exceed": int((amax.to(torch.float64) > limit).sum()),
        "ratio": float(ratios.max()),
        "source_max": float(source.abs().max()),
        "artifact_max": float(deq.abs().max()),
    }
