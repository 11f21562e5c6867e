"""HIP quantization grids vs the CPU oracle: bit-exact encodings.

Each case runs the product kernel (through the C ABI via mlx_gptq.grid) on
cuda:0 and the oracle (oracle/grid_ref.py) on the host with identical float
inputs. E8M0 / E2M1 / E4M3 / affine encodings must agree bit for bit; the
affine MSE argmin may differ only where two clip candidates' squared errors
tie to within float32 summation-order noise (checked in float64).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import grid_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    from mlx_gptq import _native

    _native.load()
    assert torch.cuda.is_available(), "GPU tests need a HIP device"


def _threshold_inputs(fmax: float) -> torch.Tensor:
    """Groups whose max|w| puts max/fmax within +-64 ulps of every E8M0 binade
    threshold, plus zeros, subnormals, inf and NaN."""
    from tests.test_oracle_closed_forms import e8m0_table

    table = e8m0_table()
    y = table.view(np.float32).astype(np.float64) * fmax
    y = y[np.isfinite(y) & (y < 3.0e38)].astype(np.float32)
    u = y.view(np.uint32).astype(np.int64)
    u = np.concatenate([b + np.arange(-64, 65) for b in u])
    u = u[(u > 0) & (u < 0x7F800000)].astype(np.uint32)
    amax = torch.from_numpy(u.view(np.float32).copy())
    extra = torch.tensor([0.0, 1e-45, 3e-39, float("inf"), float("nan"), 3.4e38], dtype=torch.float32)
    amax = torch.cat([amax, extra])
    g = torch.Generator().manual_seed(1)
    w = (torch.rand(amax.numel(), 32, generator=g) * 2 - 1) * amax.unsqueeze(1).nan_to_num(0, 0, 0)
    w[torch.arange(amax.numel()), torch.randint(0, 32, (amax.numel(),), generator=g)] = -amax
    return w


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
def test_choose_mxfp_scale_bit_exact(mode):
    from mlx_gptq import grid

    w = _threshold_inputs(grid_ref.mxfp_max(mode))
    g = torch.Generator().manual_seed(2)
    rnd = torch.randn(50000, 32, generator=g) * torch.exp(torch.randn(50000, 1, generator=g) * 8)
    for x in (w, rnd, rnd[:, :7].contiguous()):
        sb, sc = grid.choose_mxfp_scale(x.to(DEV), mode)
        rb, rs = grid_ref.choose_mxfp_scale(x, mode)
        assert torch.equal(sb.cpu(), rb)
        assert torch.equal(sc.cpu().view(torch.int32), rs.view(torch.int32))


def _e2m1_probe() -> torch.Tensor:
    thr = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0, 0.0, 1e-40], dtype=np.float32)
    u = thr.view(np.uint32).astype(np.int64)
    u = np.concatenate([b + np.arange(-4096, 4097) for b in u])
    u = u[(u >= 0) & (u < 0x7F800000)].astype(np.uint32)
    v = u.view(np.float32)
    sp = np.array([np.inf, -np.inf, np.nan, -np.nan, -0.0, 3e38], np.float32)
    return torch.from_numpy(np.concatenate([v, -v, sp]))


def _e4m3_probe() -> torch.Tensor:
    pts = [(1 + m / 16) * 2.0**e for e in range(-12, 10) for m in range(16)]
    u = np.array(pts, np.float32).view(np.uint32).astype(np.int64)
    u = np.concatenate([b + np.arange(-64, 65) for b in u]).astype(np.uint32)
    v = u.view(np.float32)
    sp = np.array([np.inf, -np.inf, np.nan, -0.0, 448.0, 464.0, 480.0, 1e-30], np.float32)
    return torch.from_numpy(np.concatenate([v, -v, sp]))


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
def test_quantize_mxfp_with_scale_bit_exact(mode):
    from mlx_gptq import grid

    x = _e2m1_probe() if mode == "mxfp4" else _e4m3_probe()
    n = x.numel() - x.numel() % 32
    w = x[:n].reshape(-1, 32).contiguous()
    ones = torch.ones(w.shape[0])
    q, dq = grid.quantize_mxfp_with_scale(w.to(DEV), ones.to(DEV), mode)
    rq, rdq = grid_ref.quantize_mxfp_with_scale(w, ones, mode)
    assert torch.equal(q.cpu(), rq)
    assert torch.equal(dq.cpu().view(torch.int32), rdq.view(torch.int32))
    # every power-of-two scale, including subnormal 2^-127 and 2^127
    g = torch.Generator().manual_seed(3)
    k = torch.randint(-127, 128, (4096,), generator=g)
    k[:2] = torch.tensor([-127, 127])
    sc = torch.pow(torch.tensor(2.0), k.float())
    w = torch.randn(4096, 32, generator=g) * sc.unsqueeze(1) * torch.exp(torch.randn(4096, 1, generator=g))
    q, dq = grid.quantize_mxfp_with_scale(w.to(DEV), sc.to(DEV), mode)
    rq, rdq = grid_ref.quantize_mxfp_with_scale(w, sc, mode)
    assert torch.equal(q.cpu(), rq)
    assert torch.equal(dq.cpu().view(torch.int32), rdq.view(torch.int32))


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
def test_dequantize_mxfp_all_codes(mode):
    from mlx_gptq import grid

    codes = torch.arange(16 if mode == "mxfp4" else 256, dtype=torch.uint8)
    q = codes.repeat(256 * 32 // codes.numel() + 1)[: 256 * 32].reshape(256, 32)
    q = q[torch.randperm(256)]
    sb = torch.arange(256, dtype=torch.uint8)
    out = grid.dequantize_mxfp(q.reshape(4, 64 * 32).to(DEV), sb.reshape(4, 64).to(DEV), mode)
    ref = grid_ref.dequantize_mxfp(q.reshape(4, 64 * 32), sb.reshape(4, 64), mode)
    assert out.shape == ref.shape
    a, b = out.cpu(), ref
    same = (a.view(torch.int32) == b.view(torch.int32)) | (torch.isnan(a) & torch.isnan(b))
    assert same.all()


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shift", [0, 1])
def test_rtn_quantize_mxfp_bit_exact(mode, dtype, shift):
    """shift = 1 hands the kernel a W that is not 16-byte aligned (the
    element-wise path); shift = 0 takes the vectorised hardware-encoder path."""
    from mlx_gptq import grid

    g = torch.Generator().manual_seed(4)
    W = (torch.randn(3, 40, 256, generator=g) * torch.exp(torch.randn(3, 40, 1, generator=g) * 3)).to(dtype)
    W[0, 0, :32] = 0.0
    W[0, 1, :4] = torch.tensor([-0.0, 1e-40, -1e-40, 0.0]).to(dtype)
    flat = torch.zeros(W.numel() + shift, dtype=dtype, device=DEV)
    Wd = flat[shift:].view(W.shape)
    Wd.copy_(W.to(DEV))
    q, sb, b, dq = grid.rtn_quantize_mxfp(Wd, mode)
    rq, rsb, rb, rdq = grid_ref.rtn_quantize_mxfp(W, mode)
    assert b is None and rb is None
    assert torch.equal(q.cpu(), rq) and torch.equal(sb.cpu(), rsb)
    assert torch.equal(dq.cpu().view(torch.int32), rdq.view(torch.int32))


def _affine_err64(w, s, b, maxq):
    s_safe = torch.where(s.abs() < 1e-12, torch.ones_like(s), s)
    q = ((w - b.unsqueeze(-1)) / s_safe.unsqueeze(-1)).round().clamp(0.0, maxq)
    dq = q * s.unsqueeze(-1) + b.unsqueeze(-1)
    return (dq.double() - w.double()).pow(2).sum(-1)


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("storage", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("G", [32, 64, 128])
def test_choose_qparams_matches_oracle(bits, storage, G):
    from mlx_gptq import grid

    g = torch.Generator().manual_seed(bits * 100 + G)
    w = torch.randn(4000, G, generator=g) * torch.exp(torch.randn(4000, 1, generator=g))
    w[0] = 0.0
    w[1] = 2.5
    w[2] = torch.linspace(-1, 1, G)
    s_st, b_st, s32, b32 = grid.choose_qparams(w.to(DEV), bits, "mse", storage)
    rs_st, rb_st, rs32, rb32 = grid_ref.choose_qparams(w, bits, "mse", storage)
    assert s_st.dtype == storage and s32.dtype == torch.float32
    diff = (s32.cpu() != rs32) | (b32.cpu() != rb32)
    # any disagreement must be a near-tie of the two candidates' squared errors
    if diff.any():
        maxq = float(2**bits - 1)
        e_gpu = _affine_err64(w[diff], s32.cpu()[diff], b32.cpu()[diff], maxq)
        e_ref = _affine_err64(w[diff], rs32[diff], rb32[diff], maxq)
        rel = (e_gpu - e_ref).abs() / e_ref.clamp_min(1e-300)
        assert (rel < 1e-5).all(), rel.max()
    assert int(diff.sum()) <= max(2, diff.numel() // 500)
    assert torch.equal(s_st.cpu()[~diff], rs_st[~diff])
    # minmax has a single candidate: always bit-exact
    s_st, b_st, s32, b32 = grid.choose_qparams(w.to(DEV), bits, "minmax", storage)
    rs_st, rb_st, rs32, rb32 = grid_ref.choose_qparams(w, bits, "minmax", storage)
    assert torch.equal(s32.cpu(), rs32) and torch.equal(b32.cpu(), rb32)


def test_quantize_with_params_and_dequant_bit_exact():
    from mlx_gptq import grid

    g = torch.Generator().manual_seed(7)
    w = torch.randn(500, 64, generator=g)
    _, _, s32, b32 = grid_ref.choose_qparams(w, 4, "mse", torch.bfloat16)
    s32[0] = 0.0
    q, dq = grid.quantize_with_params(w.to(DEV), s32.to(DEV), b32.to(DEV), 4)
    rq, rdq = grid_ref.quantize_with_params(w, s32, b32, 4)
    assert torch.equal(q.cpu(), rq) and torch.equal(dq.cpu(), rdq)
    qq = rq.to(torch.uint8).reshape(10, 50 * 64)
    s_st = s32.to(torch.bfloat16).reshape(10, 50)
    b_st = b32.to(torch.bfloat16).reshape(10, 50)
    out = grid.dequantize_artifact(qq.to(DEV), s_st.to(DEV), b_st.to(DEV), "affine", 64)
    ref = grid_ref.dequantize_artifact(qq, s_st, b_st, "affine", 64)
    assert torch.equal(out.cpu(), ref)


@pytest.mark.parametrize("bits,G", [(4, 64), (2, 32), (8, 128)])
def test_rtn_quantize_matches_oracle(bits, G):
    from mlx_gptq import grid

    g = torch.Generator().manual_seed(8)
    W = torch.randn(2, 64, 512, generator=g) * torch.rand(2, 64, 1, generator=g) * 3
    q, s, b, dq = grid.rtn_quantize(W.to(DEV), bits, G)
    rq, rs, rb, rdq = grid_ref.rtn_quantize(W, bits, G)
    same_groups = (s.cpu() == rs) & (b.cpu() == rb)
    assert same_groups.float().mean() > 0.995
    m = same_groups.unsqueeze(-1).expand(2, 64, 512 // G, G).reshape(2, 64, 512)
    assert torch.equal(q.cpu()[m], rq[m]) and torch.equal(dq.cpu()[m], rdq[m])


def test_cpu_inputs_are_staged_through_the_device():
    from mlx_gptq import grid

    W = torch.randn(8, 64)
    q, sb, _, dq = grid.rtn_quantize_mxfp(W, "mxfp4")
    assert q.device.type == "cpu"
    rq, rsb, _, rdq = grid_ref.rtn_quantize_mxfp(W, "mxfp4")
    assert torch.equal(q, rq) and torch.equal(dq, rdq)
