"""Span-batched solve of a fused expert parameter on one HIP device.

The reference solves a fused task by cutting its experts into spans that
fit a memory budget (``_expert_chunk_size``, sequential.py:314-318) and, per
span, forming each expert's Hessian from its CPU stash, stacking Hessians
and weights, and calling ``solve_gptq`` once (``one_span``,
sequential.py:546-608). Here a span costs two launch sequences: one
grouped SYRK over the routed rows already in HBM (``CaptureManager.
expert_hessians``) and one batched ``solve_gptq`` that reads the bf16 expert
weights in place. Results come back per expert, on the host, with the
metadata the reference records (tokens, rel_err, fallback).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from .capture import CaptureManager, FusedExpertTask, _hip_device
from .gptq import solve_gptq
from .grid import MX_GROUP_SIZE


def expert_bytes(C: int, R: int, mode: str = "mxfp4") -> int:
    """Device bytes one expert of a span needs: the fp32 Hessian (4 C^2),
    W_dq (4 R C), the codes (R C), the scales, and the solver workspace (per
    32-column group an fp32 U block and a compact H block, 8 KiB; the affine
    path's fp64 Cholesky workspace is 16 C^2 instead)."""
    per = 4 * C * C + 5 * R * C + R * C // MX_GROUP_SIZE * 4
    return per + (256 * C if mode in ("mxfp4", "mxfp8") else 20 * C * C)


def expert_span_size(C: int, R: int, vram_gb: float, mode: str = "mxfp4") -> int:
    """Experts per span so that one span's device buffers fit in `vram_gb`
    GiB (at least one)."""
    return max(1, int(vram_gb * (1 << 30) // expert_bytes(C, R, mode)))


@dataclass
class ExpertResult:
    expert: int
    q: torch.Tensor            # uint8 [R, C]
    scales: torch.Tensor       # [R, C / G]
    biases: torch.Tensor | None
    rel_err: float
    tokens: int
    fallback: str | None       # "all_expert_inputs" for backfilled experts


@torch.no_grad()
def solve_fused_task(
    mgr: CaptureManager,
    task: FusedExpertTask,
    bits: int,
    group_size: int,
    device="cuda",
    vram_gb: float = 64.0,
    damp: float = 0.01,
    clip: str = "mse",
    storage_dtype: torch.dtype = torch.bfloat16,
    mode: str = "affine",
    mxfp_algorithm: str = "auto",
    write_back: bool = True,
) -> list[ExpertResult]:
    """Solve every expert of `task`, span by span, on `device`.

    With ``write_back`` the dequantized weights replace the parameter's
    expert slices (as sequential.py:567 does, so the layer's re-forward sees
    the quantized experts). Returns one ``ExpertResult`` per expert, its
    tensors on the host."""
    dev = _hip_device(device)
    p = task.param
    E, R, C = (int(s) for s in p.shape)
    span = expert_span_size(C, R, vram_gb, mode)
    tokens = [mgr.stashes[k].tokens for k in task.stash_keys]
    fallback = mgr.fallback_experts
    out: list[ExpertResult] = []
    for e0 in range(0, E, span):
        e1 = min(E, e0 + span)
        H = mgr.expert_hessians(task, dev, range(e0, e1))
        W = p.detach()[e0:e1]
        if W.device != dev:
            W = W.to(dev)
        q, s, b, W_dq, rel = solve_gptq(W, H, bits, group_size, damp=damp, clip=clip,
                                        storage_dtype=storage_dtype, mode=mode,
                                        mxfp_algorithm=mxfp_algorithm)
        del H
        if write_back:
            p.data[e0:e1].copy_(W_dq.to(p.dtype))
        del W_dq
        q, s, rel = q.cpu(), s.cpu(), rel.cpu()
        b = None if b is None else b.cpu()
        for i, e in enumerate(range(e0, e1)):
            out.append(ExpertResult(e, q[i], s[i], None if b is None else b[i], float(rel[i]),
                                    tokens[e], fallback.get(task.stash_keys[e])))
    return out
