"""Range audit of calibrated artifacts against their source weights
(validate_artifacts.py:15-76), one fused device pass per tensor.

For every 32-column group the reference dequantizes the artifact and
requires max|deq| <= max(32 * max|source|, 2^-126), reporting the largest
ratio. ``range_audit`` does the dequantization, both group maxima, the
limit, the ratio and the finiteness check in one kernel
(csrc/grid.hip ``range_audit_kernel``), so neither the dequantized tensor
nor the group maxima are materialised. ``validate`` keeps the reference's
report (failures, the 20 worst ratios, status). It takes the source
tensors from a mapping or a callable rather than from a checkpoint
directory: reading checkpoint shards is the caller's side.
"""

from __future__ import annotations

import ctypes
from typing import Callable, Mapping

import torch

from . import _native as nat
from .grid import MX_GROUP_SIZE

_MODES = {"affine": 0, "mxfp4": 1, "mxfp8": 2}


def range_audit(source: torch.Tensor, q: torch.Tensor, scales: torch.Tensor, biases,
                mode: str, group_size: int) -> dict:
    """Stats of one artifact: non-finite dequantized values, groups over the
    limit, the max ratio, max|source| and max|deq|."""
    if mode not in _MODES:
        raise ValueError(f"unsupported mode {mode!r}")
    if source.dim() != 2 or tuple(source.shape) != tuple(q.shape):
        raise ValueError(f"shape {tuple(source.shape)} != {tuple(q.shape)}")
    rows, cols = source.shape
    if cols % MX_GROUP_SIZE:
        raise ValueError(f"columns {cols} not divisible by {MX_GROUP_SIZE}")
    dev = nat.device_for(source, q, scales)
    src = source
    if src.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        src = src.float()
    src = nat.on_device(src, dev)
    qq = nat.on_device(q.to(torch.uint8), dev)
    storage = 0
    if mode == "affine":
        if biases is None:
            raise ValueError("affine artifacts need biases")
        if scales.dtype != biases.dtype or scales.dtype not in (
            torch.float32, torch.bfloat16, torch.float16,
        ):
            scales, biases = scales.float(), biases.float()
        s = nat.on_device(scales.reshape(-1), dev)
        b = nat.on_device(biases.reshape(-1), dev)
        storage = nat.dtype_code(s.dtype)
    else:
        if int(group_size) != MX_GROUP_SIZE:
            raise ValueError(f"{mode} requires group size {MX_GROUP_SIZE}")
        s = nat.on_device(scales.to(torch.uint8).reshape(-1), dev)
        b = None
    stats = torch.zeros(5, dtype=torch.int64, device=dev)
    nat.call(
        "mgq_range_audit", src.data_ptr(), nat.dtype_code(src.dtype), qq.data_ptr(), s.data_ptr(),
        nat.ptr(b), storage, _MODES[mode], rows, cols, int(group_size), stats.data_ptr(),
        nat.stream_of(dev),
    )
    v = stats.cpu().numpy()
    return {
        "nonfinite": int(v[0]),
        "exceed": int(v[1]),
        "ratio": float(v[2:3].view("float64")[0]),
        "source_max": float(v[3:4].astype("uint32").view("float32")[0]),
        "artifact_max": float(v[4:5].astype("uint32").view("float32")[0]),
    }


def validate(reader, sources: Mapping[str, torch.Tensor] | Callable[[str], torch.Tensor | None],
             model_path: str = "", calib_path: str = "") -> dict:
    """The reference's report for every tensor of an ArtifactReader
    (validate_artifacts.py:21-68). ``sources`` maps a tensor name to its
    source weight (None or absent: "missing source tensor")."""
    get = sources if callable(sources) else sources.get
    failures: list[dict] = []
    worst: list[dict] = []
    for name, info in reader.tensors.items():
        source = get(name)
        if source is None:
            failures.append({"name": name, "error": "missing source tensor"})
            continue
        q, scales, biases, artifact_info = reader.get(name)
        mode = artifact_info.get("mode", info.get("mode", "affine"))
        group_size = int(artifact_info.get("group_size", info["group_size"]))
        if tuple(source.shape) != tuple(q.shape):
            failures.append({"name": name,
                             "error": f"shape {tuple(source.shape)} != {tuple(q.shape)}"})
            continue
        st = range_audit(source, q, scales, biases, mode, group_size)
        if st["nonfinite"]:
            failures.append({"name": name, "error": "non-finite dequantized values"})
            continue
        if st["exceed"]:
            failures.append({"name": name, "error": f"group range ratio {st['ratio']:.6g}"})
        worst.append({"name": name, "ratio": round(st["ratio"], 6),
                      "source_max": st["source_max"], "artifact_max": st["artifact_max"]})
    worst.sort(key=lambda item: float(item["ratio"]), reverse=True)
    return {
        "model": model_path,
        "calibration": calib_path,
        "tensors": len(reader.tensors),
        "failures": failures,
        "worst": worst[:20],
        "status": "verified" if not failures else "failed",
    }
