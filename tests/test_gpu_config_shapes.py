"""The BASELINE configs at their real sizes, checked through properties
that do not need the full CPU computation:

- Hessian: a seeded sample of entries against fp64 sums of the same bf16
  rows (relative Frobenius error over the sample <= 1e-5), exact symmetry,
  and for config 4 every expert's diagonal against fp64;
- solve: the CPU oracle on a row subset of every matrix, with the GPU's
  full Hessian, so the rows see exactly the same inputs: codes agree on
  >= 99.5 %, scales on all rows for groupwise (>= 99 % for the safe
  search), proxy loss tr((W-Q) H (W-Q)^T) of the rows within 1 %; W_dq
  decodes exactly from (q, scales);
- config 4: both Hessians' per-expert diagonals and sampled entries, the
  gate_up and down_proj solves on row samples of the lightest, median and
  heaviest experts, the unrouted experts' RTN and the whole layer's packing
  bit-exact against the oracle.

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
    _solve_vs_oracle.last = (s, W_dq)  # the full GPU result, for decision checks
    return agree, s_agree, pl, pl_ref


def _scale_gate(kw: dict) -> float:
    """Scale-byte agreement required: groupwise scales are choose_mxfp_scale
    of the original weights (gptq.py:102-106), deterministic, so every byte
    must match; the safe search's argmin over candidate objectives can flip
    at near-ties (none did on 130,944 config-4 scale bytes, 31 experts x 48
    rows of both projections), so at most one byte in a thousand may."""
    alg = kw.get("mxfp_algorithm", "auto")
    if alg == "auto":
        alg = "safe-scale-search" if kw.get("mode") == "mxfp4" else "groupwise"
    return 1.0 if alg == "groupwise" else 0.999


def _check(agree, s_agree, pl, pl_ref, s_gate=0.999):
    assert agree >= 0.995, agree
    assert s_agree >= s_gate, s_agree
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
        _check(agree, s_agree, pl, pl_ref, _scale_gate(m.solve))
        if cfg == 5 and j == 0:
            # config 5's gate_proj runs the MXFP4 safe search: its decisions
            # on 64 sampled rows x all 160 groups against float64 objectives
            s_gpu, dq_gpu = _solve_vs_oracle.last
            g = torch.Generator().manual_seed(55)
            rows = torch.sort(torch.randperm(m.W.shape[1], generator=g)[:64]).values
            cf, gf, n = _decisions_vs_fp64(m.W[0], Hs[m.inp][0], s_gpu[0], dq_gpu[0], rows)
            assert n == 64 * (m.W.shape[2] // 32)
            assert cf == 0 and gf == 0, (cf, gf, n)
            del s_gpu, dq_gpu
    del L, Hs
    torch.cuda.empty_cache()


def _decisions_vs_fp64(W, H, s, W_dq, rows, mode="mxfp4"):
    """The safe search's decisions on `rows` of one matrix (W [R, C], H
    [C, C], the solver's scale bytes s [R, C/32] and W_dq [R, C]) against the
    same decisions taken with objectives in float64 (gptq.py:107-143,164-176
    with an exact quadratic form). Returns (candidate flips, GPTQ-vs-baseline
    flips, decisions): a flip is a choice whose float64 objective exceeds the
    float64 optimum by more than 2^-18 of the sum of the magnitudes of the
    objective's terms (the size of fp32 summation error); closer calls are
    ties that any fp32 summation order may resolve either way."""
    from oracle import grid_ref

    offs = (0, -1, -2, -3, -4, 1, 2) if mode == "mxfp4" else (0, -1, 1)
    orig = W[rows].float().cpu()
    Hc = H.double().cpu()
    sk = s[rows].cpu().to(torch.int32)
    dqk = W_dq[rows].cpu()
    cand_flips = gptq_flips = 0
    n_groups = orig.shape[1] // 32
    for g in range(n_groups):
        sl = slice(32 * g, 32 * g + 32)
        o = orig[:, sl]
        Hg = Hc[sl, sl]
        e0 = grid_ref.choose_mxfp_scale(o, mode)[0].to(torch.int32) - 127
        objs, mags, dqs, bytes_ = [], [], [], []
        for off in offs:
            e = (e0 + off).clamp(-127, 127)
            _, cdq = grid_ref.quantize_mxfp_with_scale(o, torch.pow(torch.tensor(2.0), e.float()), mode)
            err = (cdq - o).double()
            objs.append(((err @ Hg) * err).sum(-1))
            mags.append(((err.abs() @ Hg.abs()) * err.abs()).sum(-1))
            dqs.append(cdq)
            bytes_.append(e + 127)
        objs, mags = torch.stack(objs), torch.stack(mags)  # [n_cand, rows]
        best, arg = objs.min(dim=0)
        pick = torch.stack(bytes_) == sk[:, g]        # candidates with the chosen byte
        inf = torch.full_like(objs, float("inf"))
        chosen, carg = torch.where(pick, objs, inf).min(dim=0)
        idx = torch.arange(len(rows))
        tol = 2.0 ** -18 * torch.maximum(mags[arg, idx], mags[carg, idx])
        cand_flips += int((chosen - best > tol).sum())
        # rows whose result is not the chosen baseline took GPTQ: its float64
        # objective must not exceed the best candidate's (the reference's <=)
        k = torch.argmax(pick.int(), dim=0)
        base = torch.stack(dqs)[k, torch.arange(len(rows))]
        took = ~(dqk[:, sl] == base).all(-1)
        err = (dqk[:, sl] - o).double()
        gobj = ((err @ Hg) * err).sum(-1)
        gmag = ((err.abs() @ Hg.abs()) * err.abs()).sum(-1)
        gtol = 2.0 ** -18 * torch.maximum(gmag, mags[carg, idx])
        gptq_flips += int((took & (gobj - chosen > gtol)).sum())
    return cand_flips, gptq_flips, n_groups * len(rows)


def _oracle_rows(W, H, q, s, W_dq, e, kw, seed, rows=48):
    """The oracle on `rows` sampled rows of expert e, with the GPU's H."""
    Ws = W[e : e + 1]
    g = torch.Generator().manual_seed(seed)
    pick = torch.sort(torch.randperm(Ws.shape[1], generator=g)[:rows]).values.to(DEV)
    Hc = H[e : e + 1].cpu()
    rq, rs, _, rW, _ = gptq_ref.solve_gptq(Ws[:, pick].cpu(), Hc.clone(), **kw)
    pl = _proxy(Ws[:, pick].float(), W_dq[e : e + 1, pick], Hc)
    pl_ref = _proxy(Ws[:, pick].float(), rW, Hc)
    _check(float((q[e : e + 1, pick].cpu() == rq).float().mean()),
           float((s[e : e + 1, pick].cpu() == rs).float().mean()), pl, pl_ref)


def test_moe_config4_full_size():
    from mlx_gptq import capture, grid, gptq, packing, synth
    from oracle import grid_ref, packing_ref

    L = synth.moe_layer(device=DEV)
    E, ne = L.experts, L.experts - L.n_empty
    Hg = capture.grouped_hessian(L.X, L.offsets, L.row_index)
    Hd = capture.grouped_hessian(L.Y, L.offsets)
    assert torch.equal(Hg, Hg.transpose(1, 2)) and torch.equal(Hd, Hd.transpose(1, 2))
    assert torch.count_nonzero(Hg[ne:]) == 0 and torch.count_nonzero(Hd[ne:]) == 0
    counts = np.array(L.counts()[:ne])
    order = np.argsort(counts, kind="stable")
    light, median, heavy = int(order[0]), int(order[ne // 2]), int(order[-1])
    # every routed expert's diagonal against fp64 sums of its gathered rows
    for e in range(ne):
        a, b = L.offsets[e], L.offsets[e + 1]
        xe = L.X.index_select(0, L.row_index[a:b].long()).double()
        ref = (xe * xe).sum(0)
        rel = float((Hg[e].diagonal().double() - ref).norm() / ref.norm())
        assert rel <= 1e-5, (e, rel)
        ye = L.Y[a:b].double()
        ref = (ye * ye).sum(0)
        rel = float((Hd[e].diagonal().double() - ref).norm() / ref.norm())
        assert rel <= 1e-5, ("down", e, rel)
    # sampled off-diagonal entries of both Hessians against fp64
    for e in sorted({0, 57, ne - 1, light, median, heavy}):
        a, b = L.offsets[e], L.offsets[e + 1]
        err = _sampled_hessian_error(L.X, Hg[e], 64, seed=e, rows=L.row_index[a:b].long())
        assert err <= 1e-5, (e, err)
        err = _sampled_hessian_error(L.Y[a:b], Hd[e], 64, seed=1000 + e)
        assert err <= 1e-5, ("down", e, err)
    # solves: all routed experts on the GPU; row samples of the light,
    # median and heavy experts (and two fixed ones) on the CPU oracle
    kw = dict(bits=4, group_size=32, mode="mxfp4")
    q, s, _, W_dq, rel = gptq.solve_gptq(L.W_gate_up[:ne], Hg[:ne], **kw)
    qd, sd, _, W_dqd, reld = gptq.solve_gptq(L.W_down[:ne], Hd[:ne], **kw)
    for e in sorted({3, ne - 2, light, median, heavy}):
        _oracle_rows(L.W_gate_up, Hg, q, s, W_dq, e, kw, seed=e)
        _oracle_rows(L.W_down, Hd, qd, sd, W_dqd, e, kw, seed=500 + e)
    for r in (rel, reld):
        assert torch.isfinite(r).all() and bool((r > 0).all())
    # the safe search decides as an exact objective would (ties aside)
    g = torch.Generator().manual_seed(4)
    for e in (light, heavy):
        for W, H, ss, dq in ((L.W_gate_up, Hg, s, W_dq), (L.W_down, Hd, sd, W_dqd)):
            rows = torch.randperm(W.shape[1], generator=g)[:64]
            cf, gf, n = _decisions_vs_fp64(W[e], H[e], ss[e], dq[e], rows)
            assert cf == 0 and gf == 0, (e, cf, gf, n)
    assert torch.equal(grid.dequantize_artifact(qd, sd, None, "mxfp4", 32), W_dqd)
    # the unrouted experts: RTN, bit-exact against the oracle
    rtn = []
    for W in (L.W_gate_up[ne:], L.W_down[ne:]):
        rq, rs, rb, rdq = grid.rtn_quantize_mxfp(W, "mxfp4")
        oq, os_, ob, odq = grid_ref.rtn_quantize_mxfp(W.cpu().float(), "mxfp4")
        assert rb is None and ob is None
        assert torch.equal(rq.cpu(), oq) and torch.equal(rs.cpu(), os_)
        assert torch.equal(rdq.cpu(), odq)
        rtn.append(rq)
    # the layer's packing: every code tensor bit-exact against the oracle
    for codes in (q, qd, *rtn):
        words = packing.pack_q(codes, 4).cpu().view(torch.int32).numpy().view(np.uint32)
        assert np.array_equal(words, packing_ref.pack_q(codes.cpu().numpy(), 4))
    # the bench's path: the solver packing its own codes gives the same codes
    # and pack_q's words for the whole gate_up layer (no routed expert has a
    # dead column, so the first solve's in-place fix left Hg as it was)
    assert bool((Hg[:ne].diagonal(dim1=1, dim2=2) > 0).all())
    packed = torch.empty(ne, q.shape[1], q.shape[2] // 8, dtype=torch.int32, device=DEV)
    q2, s2, _, W_dq2, _ = gptq.solve_gptq(L.W_gate_up[:ne], Hg[:ne], **kw, packed_out=packed)
    assert torch.equal(q2, q) and torch.equal(s2, s) and torch.equal(W_dq2, W_dq)
    assert torch.equal(packed, packing.pack_q(q, 4).view(torch.int32))
