"""HIP affine GPTQ solver (full damped Cholesky-inverse + lazy-block column
loop with the MSE clip search) vs the reference golden vectors and the CPU
oracle.

Gates: final codes agree on >= 99.5% of
elements; proxy loss tr((W-Q) H (W-Q)^T) within 1%; W_dq is exactly the
decode q*s + b of the emitted codes and stored params. The full-matrix U is
checked against an fp64 factor of the same damped matrix (the reference's
fp32 LAPACK result is within its own rounding of that) and the reference's
escalation warnings / RuntimeError are reproduced on crafted inputs.
"""

from __future__ import annotations

import logging

import pytest
import torch

from oracle import gptq_ref, hessian_ref
from tests import golden_io

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _agree(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.cpu() == b.cpu()).float().mean())


def _proxy(W, Wq, H):
    return gptq_ref.proxy_loss(W.cpu(), Wq.cpu(), H.cpu())


def _setup(B=2, R=32, C=128, N=512, seed=0, scale=1.0, outliers=0):
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(N, C, generator=g)
    X = base + 0.5 * torch.roll(base, 1, dims=1)
    X = X * torch.exp(torch.randn(C, generator=g) * 0.5)
    if outliers:
        X[:, torch.randperm(C, generator=g)[:outliers]] *= 20.0
    W = torch.randn(B, R, C, generator=g) * scale
    H = (X.T @ X).unsqueeze(0).repeat(B, 1, 1).contiguous()
    for b in range(1, B):
        H[b] *= 1.0 + 0.5 * b
    return W, H, X


def _check_vs(W, q, s, b, W_dq, rq, rs, rb, rW, H_after, min_agree=0.995):
    from mlx_gptq import grid

    G = W.shape[-1] // s.shape[-1]
    assert _agree(q, rq) >= min_agree, _agree(q, rq)
    if s.dtype == torch.float32:
        # unrounded params carry the last-ulp differences of the error
        # recurrence (reduction order of the lazy-update GEMM) straight through
        assert torch.allclose(s.cpu(), rs, rtol=1e-4, atol=0)
        assert torch.allclose(b.cpu(), rb, rtol=1e-4, atol=1e-7)
    else:
        assert _agree(s, rs) >= 0.99 and _agree(b, rb) >= 0.99
    assert torch.equal(grid.dequantize_artifact(q, s, b, "affine", G), W_dq)
    pl, pl_ref = _proxy(W, W_dq, H_after), _proxy(W, rW, H_after)
    assert torch.all((pl - pl_ref).abs() <= 0.01 * pl_ref.abs()), (pl, pl_ref)


@pytest.mark.parametrize("name", ["affine4_g64", "affine4_g32_f32", "affine2_g32",
                                  "affine8_g128_minmax"])
def test_affine_matches_reference_golden(name):
    from mlx_gptq import gptq

    t, meta = golden_io.load()
    kw = golden_io.case_kwargs(meta["cases"][name])
    W, H = t[f"{name}.W"], t[f"{name}.H"]
    Hd = H.clone().to(DEV)
    q, s, b, W_dq, rel = gptq.solve_gptq(W.to(DEV), Hd, **kw)
    assert torch.equal(Hd.cpu(), t[f"{name}.H_after"])
    assert s.dtype == t[f"{name}.scales"].dtype and b.dtype == t[f"{name}.biases"].dtype
    _check_vs(W, q, s, b, W_dq, t[f"{name}.q"], t[f"{name}.scales"], t[f"{name}.biases"],
              t[f"{name}.W_dq"], t[f"{name}.H_after"])
    assert torch.allclose(rel.cpu(), t[f"{name}.rel"], rtol=5e-3)
    # observed: every code equal to the reference's, and every rounded
    # (bf16 / f16) scale and bias; held to that
    assert torch.equal(q.cpu(), t[f"{name}.q"])
    if s.dtype != torch.float32:
        assert torch.equal(s.cpu(), t[f"{name}.scales"]) and torch.equal(b.cpu(), t[f"{name}.biases"])


@pytest.mark.parametrize("bits,G,clip,storage,block", [
    (4, 64, "mse", torch.bfloat16, 128),
    (3, 32, "mse", torch.float16, 128),
    (4, 128, "mse", torch.bfloat16, 128),
    (8, 64, "minmax", torch.bfloat16, 128),
    (4, 64, "mse", torch.bfloat16, 100),   # bs = 64 (block trimmed to a group multiple)
    (4, 32, "mse", torch.bfloat16, 512),
])
def test_affine_matches_oracle(bits, G, clip, storage, block):
    from mlx_gptq import gptq

    W, H, _ = _setup(B=2, R=96, C=384, N=2048, seed=7, scale=0.02, outliers=4)
    H[1, 50, :] = 0.0
    H[1, :, 50] = 0.0  # a dead column in one item
    Wg, Hg = W.clone().to(DEV), H.clone().to(DEV)
    q, s, b, W_dq, rel = gptq.gptq_quantize(Wg, Hg, bits, G, clip=clip, storage_dtype=storage,
                                           block_size=block)
    assert W_dq.data_ptr() == Wg.data_ptr() and rel is None
    Wr, Hr = W.clone(), H.clone()
    rq, rs, rb, rW, _ = gptq_ref.gptq_quantize(Wr, Hr, bits, G, clip=clip, storage_dtype=storage,
                                               block_size=block)
    assert torch.equal(Hg.cpu(), Hr)
    assert int(q.max()) <= 2**bits - 1
    _check_vs(W, q, s, b, W_dq, rq, rs, rb, rW, Hr)


@pytest.mark.parametrize("case,w_mult,h_mult", [
    ("tiny_H", 1.0, 1e-20),    # U's diagonal above 2^24: no RN(1/d), every error division exact-path
    ("tiny_W", 1e-31, 1.0),    # numerators below 2^-100: the error divisions leave the fast range
    ("huge_W", 1e31, 1.0),     # numerators above 2^101
])
def test_affine_out_of_range_operands_vs_oracle(case, w_mult, h_mult):
    """The column loop divides with Markstein's correction and only records
    operands outside its exact range; a group that met any is solved again
    with the guarded division. These inputs put (almost) every group on that
    second path; the codes, params and W_dq must still be the oracle's."""
    from mlx_gptq import gptq

    W, H, _ = _setup(B=2, R=64, C=256, N=1024, seed=11, scale=0.02, outliers=2)
    W = W * w_mult
    H = H * h_mult
    Wg, Hg = W.clone().to(DEV), H.clone().to(DEV)
    q, s, b, W_dq, _ = gptq.gptq_quantize(Wg, Hg, 4, 64, storage_dtype=torch.float32)
    Wr, Hr = W.clone(), H.clone()
    rq, rs, rb, rW, _ = gptq_ref.gptq_quantize(Wr, Hr, 4, 64, storage_dtype=torch.float32)
    assert torch.isfinite(W_dq).all()
    _check_vs(W, q, s, b, W_dq, rq, rs, rb, rW, Hr)


def test_affine_nonfinite_weights_leave_other_rows_on_the_oracle():
    """NaN and inf weights: a row's errors only reach that row's later
    columns, so every other row must still match the oracle. The column loop
    sends a group whose chain met a NaN or an infinity to its exact pass, and
    the clip search's ranges must not be thrown off for the rest."""
    from mlx_gptq import grid, gptq

    W, H, _ = _setup(B=2, R=64, C=256, N=1024, seed=13, scale=0.02)
    W[0, 3, 70] = float("nan")
    W[1, 10, 5] = float("inf")
    W[1, 11, 127] = -float("inf")
    W[0, 50, 200:210] = float("nan")
    Wg, Hg = W.clone().to(DEV), H.clone().to(DEV)
    q, s, b, W_dq, _ = gptq.gptq_quantize(Wg, Hg, 4, 64, storage_dtype=torch.float32)
    Wr, Hr = W.clone(), H.clone()
    rq, rs, rb, rW, _ = gptq_ref.gptq_quantize(Wr, Hr, 4, 64, storage_dtype=torch.float32)
    good = torch.isfinite(W).all(dim=-1)  # [B, R]
    assert int((~good).sum()) == 4
    q, s, b, W_dq = q.cpu(), s.cpu(), b.cpu(), W_dq.cpu()
    assert int(q.max()) <= 15
    assert _agree(q[good], rq[good]) >= 0.995
    assert torch.allclose(s[good], rs[good], rtol=1e-4, atol=0)
    assert torch.allclose(b[good], rb[good], rtol=1e-4, atol=1e-7)
    dec = grid.dequantize_artifact(q, s, b, "affine", 64)
    assert torch.equal(dec[good], W_dq[good])
    for i in range(2):
        rows = good[i]
        pl = gptq_ref.proxy_loss(W[i, rows][None], W_dq[i, rows][None], Hr[i][None])
        pl_ref = gptq_ref.proxy_loss(W[i, rows][None], rW[i, rows][None], Hr[i][None])
        assert torch.isfinite(pl).all() and (pl - pl_ref).abs() <= 0.01 * pl_ref.abs()


def test_affine_config1_shape_vs_oracle():
    """BASELINE config 1 (single Linear 2048x2048, affine 4-bit, G=64, block
    128, MSE clip) at its real size, on 8192 lognormal tokens with 1% x20
    outlier channels."""
    from mlx_gptq import gptq

    g = torch.Generator().manual_seed(17)
    C = 2048
    X = torch.randn(8192, C, generator=g) * torch.exp(torch.randn(C, generator=g))
    X[:, torch.randperm(C, generator=g)[:20]] *= 20.0
    W = (torch.randn(1, C, C, generator=g) * 0.02).to(torch.bfloat16)
    H = (X.T @ X).unsqueeze(0).contiguous()
    q, s, b, W_dq, rel = gptq.solve_gptq(W.to(DEV), H.clone().to(DEV), 4, 64)
    rq, rs, rb, rW, rrel = gptq_ref.solve_gptq(W, H.clone(), 4, 64)
    _check_vs(W.float(), q, s, b, W_dq, rq, rs, rb, rW, H)
    assert torch.allclose(rel.cpu(), rrel, rtol=1e-2)


def test_affine_config1_chain_full_size():
    """Config 1 end to end as the bench runs it: the bf16 calibration rows in
    a capture.Stash, H from Stash.hessian (the GPU SYRK), the affine solve on
    the device; against the oracle's stash Hessian of the same rows (fp32
    addmm, capture.py:68-76) and the oracle's solve."""
    from mlx_gptq import capture, gptq, synth

    L = synth.dense_config(1, device=DEV)
    X, W = L.inputs["x"], L.mats[0].W
    C = X.shape[1]
    st = capture.Stash("x", C)
    st.add(X)
    H = st.hessian(torch.device(DEV)).unsqueeze(0)
    Xc = X.cpu()
    assert hessian_ref.rel_frobenius(H[0].cpu(), hessian_ref.hessian_fp64(Xc)) < 1e-5
    q, s, b, W_dq, rel = gptq.solve_gptq(W, H.clone(), **L.mats[0].solve)
    Hr = hessian_ref.stash_hessian([Xc], C).unsqueeze(0)
    rq, rs, rb, rW, rrel = gptq_ref.solve_gptq(W.cpu(), Hr.clone(), 4, 64)
    _check_vs(W.float().cpu(), q, s, b, W_dq, rq, rs, rb, rW, Hr)
    assert torch.allclose(rel.cpu(), rrel, rtol=1e-2)


@pytest.mark.parametrize("C", [320, 200])  # 5 diagonal 64-blocks; 3 and a ragged 8-row block
def test_prepare_hinv_full_vs_fp64(C):
    from mlx_gptq import gptq

    g = torch.Generator().manual_seed(3)
    B = 3
    A = torch.randn(B, C, 2 * C, generator=g) * torch.exp(torch.randn(B, C, 1, generator=g))
    H = A @ A.transpose(1, 2)
    U = gptq._prepare_hinv(H.to(DEV), 0.01).cpu()
    assert torch.equal(U, U.triu()) and bool((U.diagonal(dim1=-2, dim2=-1) > 0).all())
    dmean = H.diagonal(dim1=-2, dim2=-1).mean(-1).clamp(min=1e-8)
    Hd = H.clone()
    Hd.diagonal(dim1=-2, dim2=-1).add_((dmean * 0.01).unsqueeze(-1))
    U64 = torch.linalg.cholesky(torch.cholesky_inverse(torch.linalg.cholesky(Hd.double())),
                                upper=True)
    rel = (U.double() - U64).norm(dim=(1, 2)) / U64.norm(dim=(1, 2))
    assert float(rel.max()) < 1e-5, rel
    Ur = gptq_ref.prepare_hinv(H.clone(), 0.01)
    rel_ref = (Ur.double() - U64).norm(dim=(1, 2)) / U64.norm(dim=(1, 2))
    assert float(rel.max()) <= float(rel_ref.max()) + 1e-6


def _indefinite(B, C, neg):
    """Diagonal-dominant SPD items with item i's diagonal entry 5 set to
    neg[i]: the damped matrix needs damp >= -neg / mean(diag) to factor."""
    g = torch.Generator().manual_seed(23)
    H = torch.zeros(B, C, C)
    for i in range(B):
        A = torch.randn(C, C, generator=g) * 0.01
        H[i] = A @ A.T + torch.eye(C)
        if neg[i] is not None:
            H[i, 5, :] = 0.0
            H[i, :, 5] = 0.0
            H[i, 5, 5] = neg[i]
    return H


def test_full_escalation_warnings_match_oracle(caplog):
    from mlx_gptq import gptq

    C = 96
    H = _indefinite(3, C, [None, -0.05, -2.0])  # needs damp 0.1 and 10
    with caplog.at_level(logging.WARNING, logger="oracle.gptq_ref"):
        events = []
        Ur = gptq_ref.prepare_hinv(H.clone(), 0.01, events=events)
    ref_msgs = [r.getMessage() for r in caplog.records]
    assert len(ref_msgs) >= 2
    caplog.clear()
    with caplog.at_level(logging.WARNING, logger="mlx_gptq.gptq"):
        U = gptq._prepare_hinv(H.to(DEV), 0.01).cpu()
    assert [r.getMessage() for r in caplog.records] == ref_msgs
    rel = (U - Ur).norm() / Ur.norm()
    assert float(rel) < 1e-4

    Hf = _indefinite(4, C, [None, -1e6, -0.05, None])  # item 1 never factors
    caplog.clear()
    with caplog.at_level(logging.WARNING, logger="oracle.gptq_ref"):
        with pytest.raises(RuntimeError) as ei_ref:
            gptq_ref.prepare_hinv(Hf.clone(), 0.01)
    ref_msgs = [r.getMessage() for r in caplog.records]
    caplog.clear()
    with caplog.at_level(logging.WARNING, logger="mlx_gptq.gptq"):
        with pytest.raises(RuntimeError) as ei:
            gptq._prepare_hinv(Hf.to(DEV), 0.01)
    assert str(ei.value) == str(ei_ref.value)
    assert [r.getMessage() for r in caplog.records] == ref_msgs


def test_solve_falls_back_when_the_first_damped_pass_fails(caplog):
    """solve_gptq launches the affine column loop before it knows the first
    damped pass succeeded. When an item needs more damping, it must solve
    again on the synchronous path: the outputs are those of gptq_quantize on
    a copy of W, with the reference's warnings; an item that never factors
    raises the reference's RuntimeError."""
    from mlx_gptq import gptq

    def coupled(B, C, off):
        # SPD items with a positive diagonal (so the dead-column fix keeps
        # them) and entries (5, 6), (6, 5) set to off[i]: the 2x2 block
        # [[1, o], [o, 1]] needs a damping above o - 1 to factor
        gg = torch.Generator().manual_seed(23)
        Hc = torch.zeros(B, C, C)
        for i in range(B):
            A = torch.randn(C, C, generator=gg) * 0.01
            Hc[i] = A @ A.T + torch.eye(C)
            if off[i] is not None:
                Hc[i, 5, 6] = Hc[i, 6, 5] = off[i]
        return Hc

    C = 128
    H = coupled(3, C, [None, 1.05, 3.0])  # needs damp 0.1 and 10
    g = torch.Generator().manual_seed(31)
    W = torch.randn(3, 48, C, generator=g) * 0.02
    with caplog.at_level(logging.WARNING, logger="mlx_gptq.gptq"):
        q, s, b, W_dq, rel = gptq.solve_gptq(W.to(DEV), H.clone().to(DEV), 4, 64)
    msgs = [r.getMessage() for r in caplog.records]
    caplog.clear()
    with caplog.at_level(logging.WARNING, logger="mlx_gptq.gptq"):
        Wc = W.clone().to(DEV)
        q2, s2, b2, W2, _ = gptq.gptq_quantize(Wc, H.clone().to(DEV), 4, 64)
    assert msgs == [r.getMessage() for r in caplog.records] and len(msgs) >= 2
    assert torch.equal(q, q2) and torch.equal(s, s2) and torch.equal(b, b2)
    assert torch.equal(W_dq, W2)
    assert torch.isfinite(rel).all()

    Hf = coupled(3, C, [None, 1e6, None])  # item 1 never factors
    caplog.clear()
    with caplog.at_level(logging.WARNING, logger="oracle.gptq_ref"):
        with pytest.raises(RuntimeError) as ei_ref:
            gptq_ref.prepare_hinv(Hf.clone(), 0.01)
    ref_msgs = [r.getMessage() for r in caplog.records]
    caplog.clear()
    with caplog.at_level(logging.WARNING, logger="mlx_gptq.gptq"):
        with pytest.raises(RuntimeError) as ei:
            gptq.solve_gptq(W.to(DEV), Hf.clone().to(DEV), 4, 64)
    assert str(ei.value) == str(ei_ref.value)
    assert [r.getMessage() for r in caplog.records] == ref_msgs


def test_solve_fallback_keeps_dead_columns_zeroed(caplog):
    """A batch where one item has dead columns (diag 0 and < 0) and another
    needs damp 0.1: the speculative first pass fails, and the synchronous
    retry must still zero the dead columns of its fresh copy of W, as the
    reference's gptq_quantize does (gptq.py:216-222) before it escalates.
    Checked against the oracle's solve_gptq on the same inputs."""
    from mlx_gptq import gptq

    C, R = 128, 48
    gg = torch.Generator().manual_seed(41)
    H = torch.zeros(3, C, C)
    for i in range(3):
        A = torch.randn(C, C, generator=gg) * 0.01
        H[i] = A @ A.T + torch.eye(C)
    H[1, 5, 6] = H[1, 6, 5] = 1.05  # needs damp 0.1 to factor
    for c, v in ((17, 0.0), (90, -2.0)):  # dead columns of item 0
        H[0, c, :] = 0.0
        H[0, :, c] = 0.0
        H[0, c, c] = v
    W = torch.randn(3, R, C, generator=gg) * 0.02
    rq, rs, rb, rW, rrel = gptq_ref.solve_gptq(W.clone(), H.clone(), 4, 64)
    Hd = H.clone().to(DEV)
    with caplog.at_level(logging.WARNING, logger="mlx_gptq.gptq"):
        q, s, b, W_dq, rel = gptq.solve_gptq(W.to(DEV), Hd, 4, 64)
    assert len(caplog.records) >= 1  # the escalation did run
    # the dead columns hold w = 0 before quantization, as in the oracle
    assert _agree(q[0, :, [17, 90]], rq[0, :, [17, 90]]) >= 0.98
    assert _agree(q[0], rq[0]) >= 0.995
    H_after = H.clone()
    H_after[0, 17, 17] = H_after[0, 90, 90] = 1.0
    assert torch.equal(Hd.cpu(), H_after)  # the dead-column fix in place, once
    _check_vs(W, q, s, b, W_dq, rq, rs, rb, rW, H_after)
    assert torch.allclose(rel.cpu(), rrel, rtol=1e-3, atol=0)


def test_affine_batched_equals_per_item():
    """Reference tests/test_gptq.py:44-52 (bit-exact), affine mode."""
    from mlx_gptq import gptq

    W, H, _ = _setup(B=3, R=40, C=256)
    qb, sb, bb, wb, _ = gptq.solve_gptq(W.to(DEV), H.clone().to(DEV), 4, 64)
    for i in range(3):
        qi, si, bi, wi, _ = gptq.solve_gptq(W[i : i + 1].to(DEV), H[i : i + 1].clone().to(DEV), 4, 64)
        assert torch.equal(qb[i], qi[0]) and torch.equal(sb[i], si[0])
        assert torch.equal(bb[i], bi[0]) and torch.equal(wb[i], wi[0])


def test_affine_gptq_improves_activation_error():
    """Reference tests/test_gptq.py:19-26."""
    from mlx_gptq import grid, gptq

    W, H, X = _setup(B=1, R=64, C=256, N=2048, seed=11)
    _, _, _, W_g, _ = gptq.solve_gptq(W.to(DEV), H.to(DEV), 4, 64)
    _, _, _, W_r = grid.rtn_quantize(W.to(DEV), 4, 64)
    e_g = ((X @ (W_g.cpu() - W).transpose(1, 2)) ** 2).mean()
    e_r = ((X @ (W_r.cpu() - W).transpose(1, 2)) ** 2).mean()
    assert e_g < e_r


def test_affine_zero_hessian_finite():
    """Reference tests/test_gptq.py:55-60."""
    from mlx_gptq import gptq

    W = torch.randn(1, 8, 128)
    H = torch.zeros(1, 128, 128)
    q, s, b, W_dq, rel = gptq.solve_gptq(W.to(DEV), H.to(DEV), 4, 64)
    assert torch.isfinite(W_dq).all()
    assert torch.count_nonzero(W_dq) == 0


def test_affine_shape_errors():
    from mlx_gptq import gptq

    W = torch.zeros(1, 4, 96, device=DEV)
    H = torch.eye(96, device=DEV).unsqueeze(0)
    with pytest.raises(AssertionError):
        gptq.gptq_quantize(W, H.clone(), 4, 64)
    with pytest.raises(AssertionError):
        gptq.gptq_quantize(W, torch.eye(64, device=DEV).unsqueeze(0), 4, 32)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
def test_rel_err_kernel_matches_the_reference_formula(dt):
    """gptq_affine.rel_err (mgq_rel_err: double partial sums, fixed order)
    against gptq.py:300-302's formula evaluated in float64 on the host; an
    all-zero original takes the 1e-12 floor of the denominator; B = 3,
    ragged n."""
    from mlx_gptq import gptq_affine

    g = torch.Generator().manual_seed(31)
    W = (torch.randn(3, 37, 1001, generator=g) * 0.02).to(dt)
    W[2] = 0
    Wdq = W.float() + torch.randn(3, 37, 1001, generator=g) * 1e-3
    got = gptq_affine.rel_err(Wdq.to(DEV), W.to(DEV)).cpu()
    W64, D64 = W.double(), Wdq.double()
    want = (D64 - W64).flatten(1).norm(dim=1) / W64.flatten(1).norm(dim=1).clamp(min=1e-12)
    assert got.dtype == torch.float32
    assert torch.allclose(got.double(), want, rtol=1e-6, atol=0)
    assert want[2] > 1e10  # the floor case
