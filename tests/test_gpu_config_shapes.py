"""The BASELINE configs at their real sizes, checked through properties
that do not need the full CPU computation:

- Hessian: a seeded sample of entries against fp64 sums of the same bf16
  rows (relative Frobenius error over the sample <= 1e-5), exact symmetry,
  and for config 4 every expert's diagonal against fp64;
- solve: the CPU oracle on a row subset of every matrix, with the GPU's
  full Hessian, so the rows see exactly the same inputs: codes agree on
  >= 99.5 %, scales on >= 99 %, proxy loss tr((W-Q) H (W-Q)^T) of the rows
  within 1 %; W_dq decodes exactly from (q, scales).

Inputs come from mlx_gptq.synth (seeded, generated on the GPU) exactly as
bench.py builds them.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gptq_ref

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _sampled_hessian_error(X: torch.Tensor, H: torch.Tensor, n_pairs: int, seed: int,
                           rows: torch.Tensor | None = None) -> float:
    """max-normalized relative Frobenius error of sampled H entries vs fp64."""
    C = X.shape[1]
    g = torch.Generator().manual_seed(seed)
    ii = torch.randint(0, C, (n_pairs,), generator=g)
    jj = torch.randint(0, C, (n_pairs,), generator=g)
    ii[:8] = jj[:8]  # a few diagonal entries
    cols = torch.unique(torch.cat([ii, jj]))
    pos = {int(c): k for k, c in enumerate(cols.tolist())}
    Xs = X[:, cols.to(X.device)] if rows is None else X.index_select(0, rows)[:, cols.to(X.device)]
    Xs = Xs.double().cpu().numpy()
    ref = np.array([Xs[:, pos[int(i)]] @ Xs[:, pos[int(j)]] for i, j in zip(ii, jj)])
    got = H[ii.to(H.device), jj.to(H.device)].double().cpu().numpy()
    return float(np.linalg.norm(got - ref) / np.linalg.norm(ref))


def _proxy(W: torch.Tensor, Wq: torch.Tensor, H: torch.Tensor) -> torch.Tensor:
    """tr((W - Q) H (W - Q)^T) per batch item in float64, computed on the GPU
    (the same quadratic form as the oracle's proxy_loss, for [*, 25600]^2)."""
    E = W.to(DEV).double() - Wq.to(DEV).double()
    Hd = H.to(DEV).double()
    return ((E @ Hd) * E).sum(dim=(1, 2)).cpu()


def _solve_vs_oracle(W: torch.Tensor, H: torch.Tensor, kw: dict, rows: int, seed: int):
    """Solve all of W on the GPU; the oracle on `rows` sampled rows."""
    from mlx_gptq import grid, gptq

    q, s, b, W_dq, rel = gptq.solve_gptq(W, H, **kw)
    R = W.shape[1]
    g = torch.Generator().manual_seed(seed)
    pick = torch.sort(torch.randperm(R, generator=g)[:rows]).values
    Hc = H.cpu()
    Ws = W[:, pick.to(W.device)].cpu()
    rq, rs, rb, rW, _ = gptq_ref.solve_gptq(Ws, Hc.clone(), **kw)
    qs, ss, Wq = q[:, pick.to(q.device)].cpu(), s[:, pick.to(s.device)].cpu(), W_dq[:, pick.to(W_dq.device)].cpu()
    agree = float((qs == rq).float().mean())
    s_agree = float((ss == rs).float().mean())
    pl = _proxy(Ws.float(), Wq, H)
    pl_ref = _proxy(Ws.float(), rW, H)
    if kw.get("mode", "affine") != "affine":
        assert torch.equal(grid.dequantize_artifact(q, s, None, kw["mode"], 32), W_dq)
    return agree, s_agree, pl, pl_ref


def _check(agree, s_agree, pl, pl_ref):
    assert agree >= 0.995, agree
    assert s_agree >= 0.99, s_agree
    assert torch.all((pl - pl_ref).abs() <= 0.01 * pl_ref.abs()), (pl, pl_ref)


@pytest.mark.parametrize("cfg", [2, 3, 5])
def test_dense_config_full_size(cfg):
    from mlx_gptq import capture, synth

    L = synth.dense_config(cfg, device=DEV)
    Hs = {}
    for k, X in L.inputs.items():
        H = capture.hessian_xtx(X)
        assert torch.equal(H, H.T)
        err = _sampled_hessian_error(X, H, 96, seed=cfg)
        assert err <= 1e-5, (cfg, k, err)
        Hs[k] = H.unsqueeze(0)
    for j, m in enumerate(L.mats):
        agree, s_agree, pl, pl_ref = _solve_vs_oracle(m.W, Hs[m.inp].clone(), m.solve, 48, seed=cfg + j)
        _check(agree, s_agree, pl, pl_ref)
    del L, Hs
    torch.cuda.empty_cache()


def test_moe_config4_full_size():
    from mlx_gptq import capture, gptq, synth

    L = synth.moe_layer(device=DEV)
    E, ne = L.experts, L.experts - L.n_empty
    Hg = capture.grouped_hessian(L.X, L.offsets, L.row_index)
    Hd = capture.grouped_hessian(L.Y, L.offsets)
    assert torch.equal(Hg, Hg.transpose(1, 2)) and torch.equal(Hd, Hd.transpose(1, 2))
    assert torch.count_nonzero(Hg[ne:]) == 0 and torch.count_nonzero(Hd[ne:]) == 0
    # every routed expert's diagonal against fp64 sums of its gathered rows
    for e in range(ne):
        a, b = L.offsets[e], L.offsets[e + 1]
        xe = L.X.index_select(0, L.row_index[a:b].long()).double()
        ref = (xe * xe).sum(0)
        rel = float((Hg[e].diagonal().double() - ref).norm() / ref.norm())
        assert rel <= 1e-5, (e, rel)
    for e in (0, 57, ne - 1):
        a, b = L.offsets[e], L.offsets[e + 1]
        err = _sampled_hessian_error(L.X, Hg[e], 64, seed=e, rows=L.row_index[a:b].long())
        assert err <= 1e-5, (e, err)
    # solve: all routed experts on the GPU, two experts' row samples on the CPU
    kw = dict(bits=4, group_size=32, mode="mxfp4")
    q, s, _, W_dq, rel = gptq.solve_gptq(L.W_gate_up[:ne], Hg[:ne], **kw)
    for e in (3, ne - 2):
        Ws = L.W_gate_up[e : e + 1]
        g = torch.Generator().manual_seed(e)
        pick = torch.sort(torch.randperm(Ws.shape[1], generator=g)[:48]).values
        Hc = Hg[e : e + 1].cpu()
        rq, rs, _, rW, _ = gptq_ref.solve_gptq(Ws[:, pick.to(DEV)].cpu(), Hc.clone(), **kw)
        qs = q[e : e + 1, pick.to(DEV)].cpu()
        ss = s[e : e + 1, pick.to(DEV)].cpu()
        pl = _proxy(Ws[:, pick.to(DEV)].float(), W_dq[e : e + 1, pick.to(DEV)], Hc)
        pl_ref = _proxy(Ws[:, pick.to(DEV)].float(), rW, Hc)
        _check(float((qs == rq).float().mean()), float((ss == rs).float().mean()), pl, pl_ref)
    assert torch.isfinite(rel).all() and bool((rel > 0).all())
