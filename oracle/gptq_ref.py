"""torch-CPU restatement of the reference GPTQ solver (test oracle only).

Follows mlx_gptq/gptq.py of the reference: dead-column fix, damped
Cholesky-inverse upper factor with per-item damping escalation, the MXFP
per-32-group solver (groupwise and safe-scale-search with the range guard),
and the affine lazy-block column loop. Same torch / LAPACK calls in the same
order as the reference, so results are the reference's bits on one build.
"""

from __future__ import annotations

import logging

import torch

from . import grid_ref as G

log = logging.getLogger("oracle.gptq_ref")

MXFP4_OFFSETS = (0, -1, -2, -3, -4, 1, 2)
MXFP8_OFFSETS = (0, -1, 1)


def prepare_hinv(H: torch.Tensor, damp: float, max_attempts: int = 6, events=None) -> torch.Tensor:
    """gptq.py:27-66. U upper with U^T U = (H + lam I)^-1, lam = damp*mean(diag).

    ``events`` (optional list) receives (n_failed, B, max_damp) per escalation
    round, the content of the reference's warning.
    """
    B, C, _ = H.shape
    dmean = H.diagonal(dim1=-2, dim2=-1).mean(dim=-1).clamp(min=1e-8)
    cur = torch.full((B,), damp, device=H.device, dtype=H.dtype)
    ar = torch.arange(C, device=H.device)
    Hd = H.clone()
    Hd[:, ar, ar] += (dmean * cur).unsqueeze(-1)
    failed = None
    ok = False
    for _ in range(max_attempts):
        L, info = torch.linalg.cholesky_ex(Hd)
        failed = info != 0
        if not failed.any():
            ok = True
            break
        cur[failed] *= 10.0
        Hd[failed] = H[failed]
        Hd[failed.nonzero(as_tuple=True)[0][:, None], ar, ar] += (dmean[failed] * cur[failed]).unsqueeze(-1)
        msg = (int(failed.sum()), B, float(cur[failed].max()))
        if events is not None:
            events.append(msg)
        log.warning("cholesky failed for %d/%d matrices, damp -> %.3g", *msg)
    if not ok:
        bad = H[failed]
        d = bad.diagonal(dim1=-2, dim2=-1)
        raise RuntimeError(
            "Hessian not positive definite after damping escalation; "
            f"batch={B} failed={int(failed.sum())} "
            f"nonfinite={int((~torch.isfinite(bad)).sum())} "
            f"diag_min={float(d.min())} diag_max={float(d.max())} "
            f"value_min={float(bad.min())} value_max={float(bad.max())}"
        )
    return torch.linalg.cholesky(torch.cholesky_inverse(L), upper=True)


def quad_form(e: torch.Tensor, Hg: torch.Tensor) -> torch.Tensor:
    """gptq.py:123-125,168: einsum('bri,bij,brj->br')."""
    return torch.einsum("bri,bij,brj->br", e, Hg, e)


def mxfp_groupwise(W, H, mode, damp, algorithm, events=None):
    """gptq.py:69-180 (W modified in place)."""
    B, R, C = W.shape
    ng = C // G.MX_GROUP_SIZE
    q_out = torch.empty(B, R, C, dtype=torch.uint8, device=W.device)
    scales = torch.empty(B, R, ng, dtype=torch.uint8, device=W.device)
    if algorithm not in ("groupwise", "safe-scale-search"):
        raise ValueError(f"unsupported MXFP GPTQ algorithm: {algorithm}")
    offsets = MXFP4_OFFSETS if mode == "mxfp4" else MXFP8_OFFSETS
    two = torch.tensor(2.0, dtype=torch.float32, device=W.device)
    for g in range(ng):
        sl = slice(g * G.MX_GROUP_SIZE, (g + 1) * G.MX_GROUP_SIZE)
        orig = W[:, :, sl].clone()
        Wg = orig.clone()
        Hg = H[:, sl, sl]
        U = prepare_hinv(Hg, damp, events=events)
        if algorithm == "groupwise":
            sbytes, svals = G.choose_mxfp_scale(orig, mode)
            base_q, base_dq = G.quantize_mxfp_with_scale(orig, svals, mode)
        else:
            e0 = G.choose_mxfp_scale(orig, mode)[0].to(torch.int32) - 127
            best = None
            for off in offsets:
                e = (e0 + off).clamp(-127, 127)
                cb = (e + 127).to(torch.uint8)
                cs = torch.pow(two, e.to(torch.float32))
                cq, cdq = G.quantize_mxfp_with_scale(orig, cs, mode)
                obj = quad_form(cdq - orig, Hg)
                if best is None:
                    best, base_q, base_dq, sbytes, svals = obj, cq, cdq, cb, cs
                else:
                    t = obj < best
                    best = torch.where(t, obj, best)
                    base_q = torch.where(t.unsqueeze(-1), cq, base_q)
                    base_dq = torch.where(t.unsqueeze(-1), cdq, base_dq)
                    sbytes = torch.where(t, cb, sbytes)
                    svals = torch.where(t, cs, svals)
        scales[:, :, g] = sbytes
        gq = torch.empty_like(orig, dtype=torch.uint8)
        gdq = torch.empty_like(orig)
        for c in range(G.MX_GROUP_SIZE):
            col = Wg[:, :, c]
            q, dq = G.quantize_mxfp_with_scale(col.unsqueeze(-1), svals, mode)
            q, dq = q.squeeze(-1), dq.squeeze(-1)
            err = (col - dq) / U[:, c, c].unsqueeze(-1)
            if c + 1 < G.MX_GROUP_SIZE:
                Wg[:, :, c + 1 :] -= err.unsqueeze(-1) * U[:, c, c + 1 :].unsqueeze(1)
            gq[:, :, c] = q
            gdq[:, :, c] = dq
        if algorithm == "groupwise":
            sel_q, sel_dq = gq, gdq
        else:
            use = quad_form(gdq - orig, Hg) <= best
            sel_q = torch.where(use.unsqueeze(-1), gq, base_q)
            sel_dq = torch.where(use.unsqueeze(-1), gdq, base_dq)
        smax = orig.abs().amax(dim=-1, keepdim=True)
        limit = torch.maximum(smax * 32.0, torch.full_like(smax, 2**-126))
        valid = (sel_dq.abs() <= limit).all(dim=-1, keepdim=True)
        q_out[:, :, sl] = torch.where(valid, sel_q, base_q)
        W[:, :, sl] = torch.where(valid, sel_dq, base_dq)
    return q_out, scales, None, W, None


@torch.no_grad()
def gptq_quantize(W, H, bits, group_size, damp=0.01, clip="mse", storage_dtype=torch.bfloat16,
                  block_size=128, mode="affine", mxfp_algorithm="auto", events=None):
    """gptq.py:183-272 (W and H modified in place)."""
    assert W.dim() == 3 and H.dim() == 3
    B, R, C = W.shape
    assert H.shape == (B, C, C)
    assert C % group_size == 0, f"in_features {C} not divisible by group {group_size}"
    if mode in ("mxfp4", "mxfp8") and group_size != G.MX_GROUP_SIZE:
        raise ValueError(f"{mode} requires group size {G.MX_GROUP_SIZE}")
    dead = H.diagonal(dim1=-2, dim2=-1) <= 0
    if dead.any():
        W[dead.unsqueeze(1).expand(B, R, C)] = 0.0
        H.diagonal(dim1=-2, dim2=-1)[dead] = 1.0
    if mode in ("mxfp4", "mxfp8"):
        if mxfp_algorithm == "auto":
            mxfp_algorithm = "safe-scale-search" if mode == "mxfp4" else "groupwise"
        return mxfp_groupwise(W, H, mode, damp, mxfp_algorithm, events=events)

    U = prepare_hinv(H, damp, events=events)
    bs = max(block_size, group_size)
    bs -= bs % group_size
    ng = C // group_size
    q_out = torch.empty(B, R, C, dtype=torch.uint8, device=W.device)
    scales = torch.empty(B, R, ng, dtype=storage_dtype, device=W.device)
    biases = torch.empty(B, R, ng, dtype=storage_dtype, device=W.device)
    s32 = b32 = None
    for i1 in range(0, C, bs):
        i2 = min(i1 + bs, C)
        n = i2 - i1
        W1 = W[:, :, i1:i2].clone()
        Err = torch.zeros(B, R, n, device=W.device)
        U1 = U[:, i1:i2, i1:i2]
        for j in range(n):
            col = i1 + j
            if col % group_size == 0:
                g = col // group_size
                s_st, b_st, s32, b32 = G.choose_qparams(W1[:, :, j : j + group_size], bits, clip, storage_dtype)
                scales[:, :, g] = s_st
                biases[:, :, g] = b_st
            w = W1[:, :, j]
            q, dq = G.quantize_with_params(w.unsqueeze(-1), s32, b32, bits)
            q, dq = q.squeeze(-1), dq.squeeze(-1)
            e = (w - dq) / U1[:, j, j].unsqueeze(-1)
            if j + 1 < n:
                W1[:, :, j + 1 :] -= e.unsqueeze(-1) * U1[:, j, j + 1 :].unsqueeze(1)
            Err[:, :, j] = e
            q_out[:, :, col] = q.to(torch.uint8)
            W[:, :, col] = dq
        if i2 < C:
            W[:, :, i2:] -= torch.bmm(Err, U[:, i1:i2, i2:])
    return q_out, scales, biases, W, None


@torch.no_grad()
def solve_gptq(W_orig, H, bits, group_size, damp=0.01, clip="mse", storage_dtype=torch.bfloat16,
               mode="affine", mxfp_algorithm="auto", events=None):
    """gptq.py:275-302."""
    W = W_orig.float().clone()
    q, s, b, W_dq, _ = gptq_quantize(W, H, bits, group_size, damp=damp, clip=clip,
                                     storage_dtype=storage_dtype, mode=mode,
                                     mxfp_algorithm=mxfp_algorithm, events=events)
    num = (W_dq - W_orig.float()).pow(2).sum(dim=(1, 2)).sqrt()
    den = W_orig.float().pow(2).sum(dim=(1, 2)).sqrt().clamp(min=1e-12)
    return q, s, b, W_dq, num / den


def proxy_loss(W, W_dq, H) -> torch.Tensor:
    """Layer proxy loss tr((W - Q) H (W - Q)^T) per batch item, in float64."""
    E = (W.double() - W_dq.double())
    return torch.einsum("bri,bij,brj->b", E, H.double(), E)
