"""Affine (MLX scale/bias) GPTQ path on the HIP kernels of csrc/chol_full.hip
and csrc/gptq_affine.hip.

  prepare_hinv_full     gptq.py:27-66 on full [C, C] Hessians: the damping
                        escalation loop (damp x10 for the failed items only,
                        up to max_attempts) around one fp64 blocked
                        factorisation pass per attempt.
  gptq_quantize_affine  gptq.py:216-272 for mode "affine": dead-column fix,
                        U, then one kernel pair per lazy block (column loop
                        with the MSE clip search at every group start, and
                        the deferred W[:, :, i2:] -= Err @ U[i1:i2, i2:]).
"""

from __future__ import annotations

import numpy as np
import torch

from . import _native as nat
from .grid import _clip_code, _storage_code


def rel_err(W_dq: torch.Tensor, W_orig: torch.Tensor) -> torch.Tensor:
    """||W_dq - W_orig||_F / max(||W_orig||_F, 1e-12) per batch item (gptq.py:300-302).

    W_dq: f32 [B, ...] on a HIP device; W_orig the weights as given (f32, bf16
    or f16 are read as they are, other dtypes as float32). One partial-sum
    launch and one reduction (mgq_rel_err), sums in double."""
    dev = W_dq.device
    W0 = W_orig.to(dev)
    if W0.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        W0 = W0.float()
    W0 = W0.contiguous()
    Wq = W_dq.contiguous()
    B = int(Wq.shape[0])
    n = int(Wq[0].numel()) if B else 0
    rel = torch.empty(B, dtype=torch.float32, device=dev)
    if B == 0:
        return rel
    nb = max(1, min(65535, -(-n // 4096)))  # about 4 K elements per partial
    part = torch.empty(B, nb, 2, dtype=torch.float64, device=dev)
    stream = nat.stream_of(dev)
    for b0 in range(0, B, 65535):  # the partial launch's grid height
        b1 = min(B, b0 + 65535)
        nat.call("mgq_rel_err", Wq[b0].data_ptr(), W0[b0].data_ptr(), nat.dtype_code(W0.dtype),
                 b1 - b0, n, part[b0].data_ptr(), nb, rel[b0:].data_ptr(), stream)
    return rel


def prepare_hinv_full(H: torch.Tensor, damp: float, max_attempts: int):
    """U [B, C, C] (f32 upper, U^T U = (H + lam I)^-1) and the attempts used per
    item (int [B], 0 = every attempt failed), for a contiguous f32 H on a HIP
    device. The reference escalates per failed item by damp *= 10 in fp32 and
    retries only those items (gptq.py:37-52); so does this loop."""
    B, C, _ = H.shape
    dev = H.device
    lib = nat.load()
    stream = nat.stream_of(dev)
    U = torch.empty(B, C, C, dtype=torch.float32, device=dev)
    attempts = np.zeros(B, dtype=np.int64)
    if B == 0 or C == 0:
        return U, attempts
    ws = torch.empty(int(lib.mgq_hinv_full_workspace_size(B, C)), dtype=torch.uint8, device=dev)
    cur = np.full(B, np.float32(damp), dtype=np.float32)
    active = np.ones(B, dtype=bool)
    for att in range(1, int(max_attempts) + 1):
        if att == 1:
            # every item, one damp: filled on the device (a host-to-device copy
            # from pageable memory would hold the host until the stream drains)
            damp_d = torch.full((B,), float(cur[0]), dtype=torch.float32, device=dev)
            active_d = torch.ones(B, dtype=torch.uint8, device=dev)
        else:
            damp_d = torch.from_numpy(cur).to(dev)
            active_d = torch.from_numpy(active.astype(np.uint8)).to(dev)
        failed_d = torch.zeros(B, dtype=torch.uint8, device=dev)
        nat.call("mgq_hinv_full_pass", H.data_ptr(), B, C, damp_d.data_ptr(), active_d.data_ptr(),
                 failed_d.data_ptr(), U.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        failed = failed_d.cpu().numpy().astype(bool) & active
        attempts[active & ~failed] = att
        if not failed.any():
            break
        cur[failed] = cur[failed] * np.float32(10.0)
        active = failed
    return U, attempts


def _first_pass_async(H: torch.Tensor, damp: float):
    """The first damped pass of prepare_hinv_full with every item active, its
    per-item failure flags copied to pinned host memory without waiting.
    Returns (U, flags, event): the flags are valid once the event has
    completed; U holds the factor of every item whose flag is 0."""
    B, C, _ = H.shape
    dev = H.device
    lib = nat.load()
    stream = nat.stream_of(dev)
    U = torch.empty(B, C, C, dtype=torch.float32, device=dev)
    ws = torch.empty(int(lib.mgq_hinv_full_workspace_size(B, C)), dtype=torch.uint8, device=dev)
    damp_d = torch.full((B,), float(np.float32(damp)), dtype=torch.float32, device=dev)
    active_d = torch.ones(B, dtype=torch.uint8, device=dev)
    failed_d = torch.zeros(B, dtype=torch.uint8, device=dev)
    nat.call("mgq_hinv_full_pass", H.data_ptr(), B, C, damp_d.data_ptr(), active_d.data_ptr(),
             failed_d.data_ptr(), U.data_ptr(), ws.data_ptr(), ws.numel(), stream)
    flags = torch.empty(B, dtype=torch.uint8, pin_memory=True)
    flags.copy_(failed_d, non_blocking=True)
    ev = torch.cuda.Event()
    ev.record(torch.cuda.current_stream(dev))
    return U, flags, ev


def gptq_quantize_affine(W: torch.Tensor, H: torch.Tensor, bits: int, group_size: int,
                         damp: float, clip: str, storage_dtype: torch.dtype, block_size: int,
                         speculative: bool = False):
    """gptq.py:216-272 for mode "affine". W f32 [B, R, C] becomes W_dq in place;
    H f32 [B, C, C] gets the dead-column diagonal fix in place.
    Returns (q u8 [B,R,C], scales, biases [B,R,C/G] storage_dtype, W, None).

    speculative: the column loop is launched right after the first damped
    pass, without waiting for its failure flags; they are read once every
    launch is queued. If some item failed, None is returned and W holds no
    meaningful result: the caller solves again from its own copy of W on the
    synchronous path, which escalates the damping and reports as the
    reference does. For callers whose W is a private copy (solve_gptq)."""
    from .gptq import _prepare_hinv, _require_device

    if W.dtype != torch.float32:
        raise TypeError("gptq_quantize updates W in place and needs float32 W")
    _require_device(W, H)
    B, R, C = W.shape
    G = int(group_size)
    bits = int(bits)
    if not 1 <= bits <= 8:
        raise ValueError(f"unsupported bits for uint8 codes: {bits}")
    if G > 128:
        raise ValueError(f"affine group size {G} unsupported on this build (<= 128)")
    storage = _storage_code(storage_dtype)
    dev = W.device
    stream = nat.stream_of(dev)
    nat.call("mgq_dead_fix", W.data_ptr(), B, R, C, H.data_ptr(), stream)
    if speculative and C != 32 and B * R * C > 0:
        U, flags, ev = _first_pass_async(H, damp)
    else:
        speculative = False
        U = _prepare_hinv(H, damp)

    bs = max(int(block_size), G)
    bs -= bs % G
    n_groups = C // G
    q_out = torch.empty(B, R, C, dtype=torch.uint8, device=dev)
    scales = torch.empty(B, R, n_groups, dtype=storage_dtype, device=dev)
    biases = torch.empty(B, R, n_groups, dtype=storage_dtype, device=dev)
    if B * R * C == 0:
        return q_out, scales, biases, W, None
    Err = torch.empty(B, R, min(bs, C), dtype=torch.float32, device=dev)
    method = _clip_code(clip)
    for i1 in range(0, C, bs):
        n = min(i1 + bs, C) - i1
        nat.call("mgq_gptq_affine_block", W.data_ptr(), U.data_ptr(), B, R, C, i1, n, G, bits,
                 method, storage, 20, 0.2, q_out.data_ptr(), scales.data_ptr(),
                 biases.data_ptr(), Err.data_ptr(), stream)
    if speculative:
        ev.synchronize()  # the first pass's flags (the blocks keep running)
        if bool(flags.any()):
            return None
    return q_out, scales, biases, W, None
