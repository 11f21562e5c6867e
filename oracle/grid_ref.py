"""torch-CPU restatement of the reference quantization grids (test oracle only).

Follows mlx_gptq/grid.py of the reference op by op: the same torch calls in
the same order, so the fp32 results are the reference's bits.
"""

from __future__ import annotations

import torch

MX_GROUP_SIZE = 32
E2M1_VALUES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0, -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0)
FMAX = {"mxfp4": 6.0, "mxfp8": 448.0}


def mxfp_max(mode: str) -> float:
    """grid.py:53-58."""
    if mode not in FMAX:
        raise ValueError(f"not a microscaling mode: {mode}")
    return FMAX[mode]


def choose_mxfp_scale(w: torch.Tensor, mode: str):
    """grid.py:61-79: e = clamp(round(log2(max|w| / fmax)), -127, 127), 0 if max = 0."""
    fmax = mxfp_max(mode)
    amax = w.abs().amax(dim=-1)
    zero = amax == 0
    y = torch.where(zero, torch.full_like(amax, fmax), amax) / fmax
    e = torch.round(torch.log2(y)).to(torch.int32).clamp(-127, 127)
    e = torch.where(zero, torch.zeros_like(e), e)
    two = torch.tensor(2.0, dtype=torch.float32, device=w.device)
    return (e + 127).to(torch.uint8), torch.pow(two, e.to(torch.float32))


def e2m1_codes(x: torch.Tensor) -> torch.Tensor:
    """grid.py:82-105: magnitude thresholds with alternating strictness (RNE on
    the E2M1 grid), sign bit for x < 0 only."""
    ax = x.abs()
    mag = torch.zeros(x.shape, dtype=torch.uint8, device=x.device)
    # (threshold, strict, code): applied from the smallest threshold up, each
    # later hit overwrites, which equals the reference's nested where chain.
    for thr, strict, code in (
        (0.25, True, 1), (0.75, False, 2), (1.25, True, 3), (1.75, False, 4),
        (2.5, True, 5), (3.5, False, 6), (5.0, True, 7),
    ):
        hit = ax > thr if strict else ax >= thr
        mag = torch.where(hit, torch.full_like(mag, code), mag)
    return mag | ((x < 0).to(torch.uint8) << 3)


def quantize_mxfp_with_scale(w: torch.Tensor, scales: torch.Tensor, mode: str):
    """grid.py:108-124."""
    n = w / scales.unsqueeze(-1)
    if mode == "mxfp4":
        q = e2m1_codes(n)
        lut = torch.tensor(E2M1_VALUES, dtype=torch.float32, device=w.device)
        return q, lut[q.to(torch.long)] * scales.unsqueeze(-1)
    if mode == "mxfp8":
        f8 = n.clamp(-448.0, 448.0).contiguous().to(torch.float8_e4m3fn).contiguous()
        return f8.view(torch.uint8), f8.float() * scales.unsqueeze(-1)
    raise ValueError(f"not a microscaling mode: {mode}")


def dequantize_mxfp(q: torch.Tensor, scale_bytes: torch.Tensor, mode: str):
    """grid.py:127-139 -> [..., C/32, 32]."""
    two = torch.tensor(2.0, dtype=torch.float32, device=q.device)
    sc = torch.pow(two, scale_bytes.to(torch.float32) - 127.0)
    if mode == "mxfp4":
        v = torch.tensor(E2M1_VALUES, dtype=torch.float32, device=q.device)[q.to(torch.long)]
    elif mode == "mxfp8":
        v = q.contiguous().view(torch.float8_e4m3fn).float()
    else:
        raise ValueError(f"not a microscaling mode: {mode}")
    return v.reshape(*q.shape[:-1], -1, MX_GROUP_SIZE) * sc.unsqueeze(-1)


@torch.no_grad()
def rtn_quantize_mxfp(W: torch.Tensor, mode: str):
    """grid.py:142-151."""
    *lead, R, C = W.shape
    if C % MX_GROUP_SIZE:
        raise ValueError(f"columns {C} not divisible by {MX_GROUP_SIZE}")
    g = W.reshape(*lead, R, C // MX_GROUP_SIZE, MX_GROUP_SIZE).float()
    sb, sc = choose_mxfp_scale(g, mode)
    q, dq = quantize_mxfp_with_scale(g, sc, mode)
    return q.reshape(*lead, R, C), sb, None, dq.reshape(*lead, R, C)


def dequantize_artifact(q, scales, biases, mode: str, group_size: int):
    """grid.py:154-164."""
    if mode == "affine":
        qq = q.to(torch.float32).reshape(*q.shape[:-1], -1, group_size)
        return (qq * scales.float().unsqueeze(-1) + biases.float().unsqueeze(-1)).reshape(q.shape)
    if group_size != MX_GROUP_SIZE:
        raise ValueError(f"{mode} requires group size {MX_GROUP_SIZE}")
    return dequantize_mxfp(q, scales, mode).reshape(q.shape)


def shrink_factors(method: str, grid_steps: int = 20, max_shrink: float = 0.2) -> list[float]:
    """grid.py:189-192 (Python doubles)."""
    if method == "minmax":
        return [1.0]
    return [1.0 - max_shrink * i / grid_steps for i in range(grid_steps + 1)]


def affine_candidate(w, wmin, wmax, p, maxq, storage_dtype):
    """One clip candidate of grid.py:196-203 -> (s, b, err)."""
    s = ((wmax - wmin) * (p / maxq)).to(storage_dtype).float()
    b = (wmin * p).to(storage_dtype).float()
    s_safe = torch.where(s.abs() < 1e-12, torch.ones_like(s), s)
    q = ((w - b.unsqueeze(-1)) / s_safe.unsqueeze(-1)).round_().clamp_(0.0, maxq)
    dq = q * s.unsqueeze(-1) + b.unsqueeze(-1)
    return s, b, (dq - w).pow(2).sum(dim=-1)


def choose_qparams(w, bits, method="mse", storage_dtype=torch.bfloat16, grid_steps=20, max_shrink=0.2):
    """grid.py:167-212: strict-< argmin over the shrink candidates."""
    maxq = float(2**bits - 1)
    wmin, wmax = w.amin(dim=-1), w.amax(dim=-1)
    best = None
    for p in shrink_factors(method, grid_steps, max_shrink):
        s, b, err = affine_candidate(w, wmin, wmax, p, maxq, storage_dtype)
        if best is None:
            best = [err, s, b]
            continue
        take = err < best[0]
        best = [torch.where(take, err, best[0]), torch.where(take, s, best[1]), torch.where(take, b, best[2])]
    _, s, b = best
    return s.to(storage_dtype), b.to(storage_dtype), s.float(), b.float()


def quantize_with_params(w, s32, b32, bits):
    """grid.py:215-221."""
    maxq = float(2**bits - 1)
    s_safe = torch.where(s32.abs() < 1e-12, torch.ones_like(s32), s32)
    q = ((w - b32.unsqueeze(-1)) / s_safe.unsqueeze(-1)).round_().clamp_(0.0, maxq)
    return q, q * s32.unsqueeze(-1) + b32.unsqueeze(-1)


@torch.no_grad()
def rtn_quantize(W, bits, group_size, method="mse", storage_dtype=torch.bfloat16):
    """grid.py:224-246."""
    *lead, R, C = W.shape
    assert C % group_size == 0, f"cols {C} not divisible by group size {group_size}"
    g = W.reshape(*lead, R, C // group_size, group_size).float()
    s_st, b_st, s32, b32 = choose_qparams(g, bits, method, storage_dtype)
    q, dq = quantize_with_params(g, s32, b32, bits)
    return q.to(torch.uint8).reshape(*lead, R, C), s_st, b_st, dq.reshape(*lead, R, C)
