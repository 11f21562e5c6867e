"""Batched GPTQ solver on MI355X behind the reference solver API.

Same entry points, arguments, defaults, return tuples, in-place semantics,
warnings and exceptions as the reference module mlx_gptq/gptq.py:

  _prepare_hinv(H, damp, max_attempts=6)                      gptq.py:27-66
  _gptq_quantize_mxfp_groupwise(W, H, mode, damp, algorithm)  gptq.py:69-180
  gptq_quantize(W, H, bits, group_size, ...)                  gptq.py:183-272
  solve_gptq(W_orig, H, bits, group_size, ...)                gptq.py:275-302

W is [B, out, in] (B = batched experts, 1 for a dense linear), H is
[B, in, in]. The arithmetic runs in the HIP kernels of libmlxgptq_hip.so
(csrc/cholesky.hip, csrc/gptq_mxfp.hip, csrc/gptq_affine.hip); this module
validates arguments, allocates outputs/workspace with torch on the tensors'
device, reproduces the reference's damping-escalation warnings from the
per-block attempt counts the kernels report, and raises its RuntimeError.
"""

from __future__ import annotations

import ctypes
import logging

import numpy as np
import torch

from . import _native as nat
from .grid import MX_GROUP_SIZE

log = logging.getLogger(__name__)

MXFP4_OFFSETS = (0, -1, -2, -3, -4, 1, 2)
MXFP8_OFFSETS = (0, -1, 1)


def _escalation_report(attempts: np.ndarray, B: int, damp: float, max_attempts: int,
                       H_blocks) -> None:
    """Emit the reference's per-round warnings for one _prepare_hinv call and
    raise its RuntimeError if some block never factorised (gptq.py:37-63).

    attempts: int [B] (attempts used, 0 = failed every attempt).
    H_blocks: callable(failed_index_array) -> float tensor [F, n, n] of the
    undamped blocks, used only for the failure message.
    """
    failed_all = attempts == 0
    rounds = max_attempts if failed_all.any() else int(attempts.max()) - 1
    cur = np.float32(damp)
    for r in range(max(rounds, 0)):
        cur = np.float32(cur * np.float32(10.0))
        failed = failed_all | (attempts > r + 1)
        log.warning("cholesky failed for %d/%d matrices, damp -> %.3g", int(failed.sum()), B, float(cur))
    if failed_all.any():
        bad = H_blocks(np.nonzero(failed_all)[0])
        diag = bad.diagonal(dim1=-2, dim2=-1)
        raise RuntimeError(
            "Hessian not positive definite after damping escalation; "
            f"batch={B} failed={int(failed_all.sum())} "
            f"nonfinite={int((~torch.isfinite(bad)).sum())} "
            f"diag_min={float(diag.min())} diag_max={float(diag.max())} "
            f"value_min={float(bad.min())} value_max={float(bad.max())}"
        )


def _prepare_hinv(H: torch.Tensor, damp: float, max_attempts: int = 6) -> torch.Tensor:
    """Upper Cholesky factor of (H + damp*mean(diag)*I)^-1, batched, with
    per-item damping escalation (gptq.py:27-66). H: float32 [B, C, C]."""
    B, C, _ = H.shape
    dev = nat.device_for(H)
    Hc = nat.on_device(H.float(), dev)
    if C == MX_GROUP_SIZE:
        U = torch.empty(B, C, C, dtype=torch.float32, device=dev)
        att = torch.empty(B, dtype=torch.int32, device=dev)
        nat.call("mgq_prepare_hinv_blocks", Hc.data_ptr(), B, C, C, float(damp),
                 int(max_attempts), U.data_ptr(), att.data_ptr(), nat.stream_of(dev))
    else:
        from . import gptq_affine

        U, att = gptq_affine.prepare_hinv_full(Hc.contiguous(), damp, max_attempts)
    att = att if isinstance(att, np.ndarray) else att.cpu().numpy()
    _escalation_report(att, B, damp, max_attempts, lambda idx: Hc[torch.as_tensor(idx, device=dev)])
    return U.to(H.device)


def _mxfp_solve(W_in: torch.Tensor, H: torch.Tensor, mode: str, damp: float, algorithm: str,
                W_out: torch.Tensor, want_rel: bool, packed: torch.Tensor | None = None):
    """Launch the fused MXFP solver; returns (q, scales, rel|None).
    packed (u32/i32 [B, R, C * bits / 32], bits 4 for mxfp4 and 8 for mxfp8):
    also filled with pack_q(q, bits) (packing.py:15-26) by the solver.

    The damped Cholesky-inverse runs first (mgq_gptq_mxfp_prepare); its
    per-block attempt counts are copied to pinned host memory before the
    group solver is launched, so the reference's warnings and RuntimeError
    (gptq.py:37-63) come from a short wait for that copy instead of a wait
    for the whole solve. In place (W_out is W_in) the solver is only launched
    once the attempts are known, so a failing call leaves W untouched as the
    reference's does."""
    if algorithm not in ("groupwise", "safe-scale-search"):
        raise ValueError(f"unsupported MXFP GPTQ algorithm: {algorithm}")
    B, R, C = W_in.shape
    dev = W_out.device
    q = torch.empty(B, R, C, dtype=torch.uint8, device=dev)
    scales = torch.empty(B, R, C // MX_GROUP_SIZE, dtype=torch.uint8, device=dev)
    rel = torch.empty(B, dtype=torch.float32, device=dev) if want_rel else None
    att = torch.empty(C // MX_GROUP_SIZE, B, dtype=torch.int32, device=dev)
    lib = nat.load()
    ws = torch.empty(int(lib.mgq_gptq_mxfp_workspace_size(B, R, C)), dtype=torch.uint8, device=dev)
    offs = MXFP4_OFFSETS if mode == "mxfp4" else MXFP8_OFFSETS
    offs_arr = (ctypes.c_int32 * len(offs))(*offs)  # alive until the call returns
    stream = nat.stream_of(dev)
    nat.call("mgq_gptq_mxfp_prepare", H.data_ptr(), B, R, C, float(damp), 6, att.data_ptr(),
             ws.data_ptr(), ws.numel(), stream)

    def solve():
        head = (W_in.data_ptr(), nat.dtype_code(W_in.dtype), B, R, C, nat.mode_code(mode),
                1 if algorithm == "safe-scale-search" else 0, ctypes.addressof(offs_arr), len(offs),
                q.data_ptr())
        tail = (scales.data_ptr(), W_out.data_ptr(), None if rel is None else rel.data_ptr(),
                ws.data_ptr(), ws.numel(), stream)
        if packed is None:
            nat.call("mgq_gptq_mxfp_solve", *head, *tail)
        else:
            nat.call("mgq_gptq_mxfp_solve_packed", *head, packed.data_ptr(), *tail)

    if W_out.data_ptr() == W_in.data_ptr():
        att_h = att.cpu().numpy()
        _attempts_report(att_h, B, damp, H, dev)
        solve()
        return q, scales, rel
    att_host = torch.empty(att.shape, dtype=torch.int32, pin_memory=True)
    att_host.copy_(att, non_blocking=True)
    copied = torch.cuda.Event()
    copied.record(torch.cuda.current_stream(dev))
    solve()
    copied.synchronize()
    _attempts_report(att_host.numpy(), B, damp, H, dev)
    return q, scales, rel


def _attempts_report(att_h: np.ndarray, B: int, damp: float, H: torch.Tensor, dev) -> None:
    """Warnings / RuntimeError of every 32-column group's _prepare_hinv call."""
    if att_h.size == 0 or (att_h.min() == 1 and att_h.max() == 1):
        return  # every block factored at the first damping: nothing to report
    for g in range(att_h.shape[0]):
        sl = slice(g * MX_GROUP_SIZE, (g + 1) * MX_GROUP_SIZE)
        _escalation_report(att_h[g], B, damp, 6,
                           lambda idx, sl=sl: H[torch.as_tensor(idx, device=dev)][:, sl, sl])


def _staged(W: torch.Tensor, H: torch.Tensor, w_dtype: torch.dtype | None = None):
    """(W_d, H_d): W and H on the HIP device that solves them -- the one
    either already lives on, else the current device -- contiguous, H in
    float32 (W in ``w_dtype`` if given). Tensors that already qualify are
    returned as they are, so in-place updates land in the caller's tensors;
    the caller copies results back into the others. Raises if no HIP device
    is visible: nothing here computes on the host."""
    dev = nat.device_for(W, H)
    if W.is_cuda and H.is_cuda and W.device != H.device:
        raise RuntimeError(f"W on {W.device} but H on {H.device}")

    def put(t, dt):
        # the kernels read 16-byte pieces: a misaligned tensor is staged too
        if t.device == dev and t.dtype == dt and t.is_contiguous() and t.data_ptr() % 16 == 0:
            return t
        return t.to(device=dev, dtype=dt, copy=True).contiguous()

    return put(W, w_dtype or W.dtype), put(H, torch.float32)


@torch.no_grad()
def _gptq_quantize_mxfp_groupwise(W: torch.Tensor, H: torch.Tensor, mode: str, damp: float,
                                  algorithm: str):
    """GPTQ independently inside each native 32-value group (gptq.py:69-180).

    W float32 [B, R, C] is overwritten with the dequantized weights.
    Returns (q uint8, scales uint8 E8M0, None, W, None).
    """
    if algorithm not in ("groupwise", "safe-scale-search"):
        raise ValueError(f"unsupported MXFP GPTQ algorithm: {algorithm}")
    W_d, H_d = _staged(W, H)
    _require_device(W_d, H_d)
    q, scales, _ = _mxfp_solve(W_d, H_d, mode, damp, algorithm, W_d, False)
    _write_back(W, W_d, H, H_d)
    return q.to(W.device), scales.to(W.device), None, W, None


def _write_back(W, W_d, H, H_d) -> None:
    """Copy the in-place results (W_dq, the dead-column diagonals of H) from
    the solving device's copies into the caller's tensors."""
    if W_d is not W:
        W.copy_(W_d)
    if H_d is not H:
        H.copy_(H_d)


def _require_device(W: torch.Tensor, H: torch.Tensor) -> None:
    nat.device_for(W, H)
    if not (W.is_cuda and H.is_cuda):
        raise RuntimeError(
            "mlx_gptq (MI355X build) solves on HIP devices only; move W and H to a "
            "cuda (HIP) device first"
        )
    if W.device != H.device:
        raise RuntimeError(f"W on {W.device} but H on {H.device}")
    if H.dtype != torch.float32 or not H.is_contiguous():
        raise TypeError("H must be a contiguous float32 tensor")
    if not W.is_contiguous():
        raise TypeError("W must be contiguous")


@torch.no_grad()
def gptq_quantize(
    W: torch.Tensor,
    H: torch.Tensor,
    bits: int,
    group_size: int,
    damp: float = 0.01,
    clip: str = "mse",
    storage_dtype: torch.dtype = torch.bfloat16,
    block_size: int = 128,
    mode: str = "affine",
    mxfp_algorithm: str = "auto",
):
    """Quantize W (in-place error compensation) against Hessian H (gptq.py:183-272).

    W: [B, out, in] float32 (overwritten with the dequantized weights),
    H: [B, in, in] float32 (dead-column diagonals set to 1 in place).
    Returns (q uint8, scales, biases | None, W_dq (= W), None).

    W and H may live on the host (dflash2_calibrate.py:55-80 solves large
    matrices from CPU tensors): they are solved on the current HIP device and
    the results come back to W's device, W and H updated in place.
    """
    assert W.dim() == 3 and H.dim() == 3
    B, R, C = W.shape
    assert H.shape == (B, C, C)
    assert C % group_size == 0, f"in_features {C} not divisible by group {group_size}"
    if mode in ("mxfp4", "mxfp8") and group_size != MX_GROUP_SIZE:
        raise ValueError(f"{mode} requires group size {MX_GROUP_SIZE}")
    if W.dtype != torch.float32:
        raise TypeError("gptq_quantize updates W in place and needs float32 W")
    if mode in ("mxfp4", "mxfp8"):
        if mxfp_algorithm == "auto":
            mxfp_algorithm = "safe-scale-search" if mode == "mxfp4" else "groupwise"
        return _gptq_quantize_mxfp_groupwise(W, H, mode, damp, mxfp_algorithm)
    # any other mode string takes the affine path, as in the reference
    from . import gptq_affine

    W_d, H_d = _staged(W, H)
    q, s, b, _, _ = gptq_affine.gptq_quantize_affine(W_d, H_d, bits, group_size, damp, clip,
                                                     storage_dtype, block_size)
    _write_back(W, W_d, H, H_d)
    return q.to(W.device), s.to(W.device), b.to(W.device), W, None


@torch.no_grad()
def solve_gptq(
    W_orig: torch.Tensor,
    H: torch.Tensor,
    bits: int,
    group_size: int,
    damp: float = 0.01,
    clip: str = "mse",
    storage_dtype: torch.dtype = torch.bfloat16,
    mode: str = "affine",
    mxfp_algorithm: str = "auto",
    *,
    packed_out: torch.Tensor | None = None,
):
    """Keep W_orig intact, return (q, scales, biases, W_dq, rel_err[B]) (gptq.py:275-302).

    Host tensors are solved on the current HIP device; every output is
    returned on W_orig's device and H gets the dead-column fix in place,
    as the reference's device-agnostic torch code does.

    packed_out (keyword only, not in the reference's signature): a
    contiguous uint32 / int32 tensor [B, out, in * pack_bits / 32] on the
    solving device, filled with ``packing.pack_q(q, pack_bits)``
    (packing.py:15-26), pack_bits 4 for mxfp4, 8 for mxfp8 and ``bits`` for
    the affine modes. The MXFP solver writes it from the codes it holds,
    so the codes are not read back for a separate packing pass."""
    out_dev = W_orig.device
    if mode in ("mxfp4", "mxfp8"):
        assert W_orig.dim() == 3 and H.dim() == 3
        B, R, C = W_orig.shape
        assert H.shape == (B, C, C)
        assert C % group_size == 0, f"in_features {C} not divisible by group {group_size}"
        if group_size != MX_GROUP_SIZE:
            raise ValueError(f"{mode} requires group size {MX_GROUP_SIZE}")
        if mxfp_algorithm == "auto":
            mxfp_algorithm = "safe-scale-search" if mode == "mxfp4" else "groupwise"
        # bf16 / f16 weights are read as they are (their float() is exact)
        wdt = W_orig.dtype if W_orig.dtype in (torch.float32, torch.bfloat16, torch.float16) \
            else torch.float32
        src, H_d = _staged(W_orig, H, wdt)
        _require_device(src, H_d)
        if packed_out is not None:
            _check_packed(packed_out, (B, R, C), 4 if mode == "mxfp4" else 8, src.device)
        W_dq = torch.empty(B, R, C, dtype=torch.float32, device=src.device)
        q, s, rel = _mxfp_solve(src, H_d, mode, damp, mxfp_algorithm, W_dq, True, packed_out)
        if H_d is not H:
            H.copy_(H_d)
        return q.to(out_dev), s.to(out_dev), None, W_dq.to(out_dev), rel.to(out_dev)
    from . import gptq_affine

    W0, H_d = _staged(W_orig, H)
    assert W0.dim() == 3 and H_d.dim() == 3
    B, R, C = W0.shape
    assert H_d.shape == (B, C, C)
    assert C % group_size == 0, f"in_features {C} not divisible by group {group_size}"
    if packed_out is not None:
        _check_packed(packed_out, (B, R, C), bits, W0.device)
    # W is a private copy, so the column loop may start before the first
    # damped pass is known to have succeeded; if it had not, solve again from
    # a fresh copy on the synchronous path (escalation, warnings, errors).
    # The speculative pass has already given H_d's dead columns (diag <= 0)
    # a unit diagonal, so the retry would no longer see them: their mask is
    # kept from before, and the retry's copy of W gets those columns zeroed
    # as the reference's dead-column fix does (gptq.py:216-222).
    dead = torch.diagonal(H_d, dim1=-2, dim2=-1) <= 0
    W = W0.to(torch.float32, copy=True)
    res = gptq_affine.gptq_quantize_affine(W, H_d, bits, group_size, damp, clip, storage_dtype,
                                           128, speculative=True)
    if res is None:
        W = W0.to(torch.float32, copy=True)
        W.masked_fill_(dead.unsqueeze(1), 0.0)
        res = gptq_quantize(W, H_d, bits, group_size, damp=damp, clip=clip,
                            storage_dtype=storage_dtype, mode=mode, mxfp_algorithm=mxfp_algorithm)
    q, s, b, W_dq, _ = res
    rel = gptq_affine.rel_err(W_dq, W0)
    if H_d is not H:
        H.copy_(H_d)
    if packed_out is not None:
        nat.call("mgq_pack_q", q.data_ptr(), B * R, C, bits, packed_out.data_ptr(),
                 nat.stream_of(q.device))
    return q.to(out_dev), s.to(out_dev), b.to(out_dev), W_dq.to(out_dev), rel.to(out_dev)


def _check_packed(packed: torch.Tensor, shape, pack_bits: int, dev) -> None:
    B, R, C = shape
    if pack_bits not in (2, 4, 8) or C % (32 // pack_bits):
        raise ValueError(f"cannot pack {pack_bits}-bit codes of {C} columns for MLX")
    want = (B, R, C * pack_bits // 32)
    if (packed.dtype not in (torch.int32, getattr(torch, "uint32", torch.int32))
            or tuple(packed.shape) != want or not packed.is_contiguous()
            or packed.device != dev or packed.data_ptr() % 16):
        raise ValueError(f"packed_out must be a contiguous 16-byte aligned uint32 / int32 "
                         f"tensor {list(want)} on {dev}")
