"""Pin the CPU oracle (and the product's E8M0 table) against what the
mathematics or a library routine fixes, independently of the restatement.

- E8M0: the generated binade-threshold table vs torch's own log2/round at
  +-64 ulps of every threshold; the oracle vs that closed form.
- E2M1: nearest-value-with-even-tie on the grid, computed in float64.
- E4M3: round-half-even onto the e4m3fn grid, computed in float64.
- packing: the reference's known answer (tests/test_dflash2_pack.py:6-11)
  and the little-endian equivalence of uint32 and nibble packing
  (tests/test_grid_and_packing.py:61-72).
- Hessian: X^T X against float64.
- Cholesky-inverse: uniqueness invariants of the upper factor.
"""

from __future__ import annotations

import os
import re

import numpy as np
import pytest
import torch

from oracle import gptq_ref, grid_ref, hessian_ref, packing_ref

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TABLE_H = os.path.join(ROOT, "mlx-gptq-mxfp_amd", "csrc", "e8m0_thresholds.h")


def e8m0_table() -> np.ndarray:
    txt = open(TABLE_H).read()
    body = txt[txt.index("{") + 1 : txt.index("};")]
    vals = [int(v, 16) for v in re.findall(r"0x([0-9a-f]+)u", body)]
    assert len(vals) == 255
    return np.array(vals, dtype=np.uint32)


def e8m0_closed_form(y_bits: np.ndarray, table: np.ndarray) -> np.ndarray:
    """Exponent from the fp32 bit pattern of y = max|w| / fmax (finite, > 0)."""
    u = y_bits.astype(np.int64)
    out = np.empty(u.shape, dtype=np.int64)
    sub = u < 0x00800000
    out[sub] = np.where(u[sub] >= table[0], -126, -127)
    e = (u[~sub] >> 23) - 127
    t = table[np.clip(e + 1 + 126, 0, 254)]
    out[~sub] = np.minimum(e + (u[~sub] >= t), 127)
    return out


def test_e8m0_table_matches_torch_log2_round():
    table = e8m0_table()
    ys = []
    for T in table:
        ys.append(np.arange(-64, 65, dtype=np.int64) + int(T))
    u = np.concatenate(ys)
    u = u[(u > 0) & (u < 0x7F800000)].astype(np.uint32)
    y = torch.from_numpy(u.view(np.float32).copy())
    e_torch = torch.round(torch.log2(y)).to(torch.int32).clamp(-127, 127).numpy()
    np.testing.assert_array_equal(e8m0_closed_form(u, table), e_torch)


@pytest.mark.parametrize("mode", ["mxfp4", "mxfp8"])
def test_oracle_e8m0_matches_closed_form(mode):
    table = e8m0_table()
    g = torch.Generator().manual_seed(5)
    # magnitudes spanning the whole fp32 range, plus subnormals and zeros
    mant = torch.rand(20000, generator=g) + 1.0
    expo = torch.randint(-149, 128, (20000,), generator=g).to(torch.float32)
    amax = (mant * torch.pow(2.0, expo)).clamp(max=3.0e38)
    amax[:50] = 0.0
    amax[50:100] = torch.rand(50, generator=g) * 1e-40
    w = torch.zeros(20000, 32)
    w[:, 7] = -amax
    sb, sc = grid_ref.choose_mxfp_scale(w, mode)
    fmax = np.float32(grid_ref.mxfp_max(mode))
    y = (amax.numpy() / fmax).astype(np.float32)
    exp = e8m0_closed_form(y.view(np.uint32), table)
    exp = np.where(amax.numpy() == 0, 0, exp)
    np.testing.assert_array_equal(sb.numpy().astype(np.int64) - 127, exp)
    np.testing.assert_array_equal(sc.numpy(), np.ldexp(np.float32(1.0), exp.astype(np.int32)).astype(np.float32))


def _e2m1_expected(x: np.ndarray) -> np.ndarray:
    grid = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])
    ax = np.abs(x.astype(np.float64))
    d = np.abs(ax[:, None] - grid[None, :])
    best = d.min(axis=1, keepdims=True)
    tie = d == best
    # nearest value; on a tie the even code (RNE in code space); saturate above 6
    idx = np.where(tie.sum(1) > 1, np.argmax(tie & (np.arange(8) % 2 == 0)[None, :], axis=1), np.argmin(d, axis=1))
    idx = np.where(ax > 6.0, 7, idx)  # saturate (also for inf and huge values)
    idx = np.where(np.isnan(ax), 0, idx)
    sign = (x < 0).astype(np.int64) << 3
    return (idx | sign).astype(np.uint8)


def test_oracle_e2m1_matches_closed_form():
    thr = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0, 0.0], dtype=np.float32)
    bits = thr.view(np.uint32).astype(np.int64)
    u = np.concatenate([b + np.arange(-256, 257) for b in bits])
    u = u[(u >= 0) & (u < 0x7F800000)].astype(np.uint32)
    vals = u.view(np.float32)
    rng = np.random.default_rng(3)
    rnd = (rng.standard_normal(100000) * 4).astype(np.float32)
    x = np.concatenate([vals, -vals, rnd, np.array([np.inf, -np.inf, np.nan, -0.0, 1e30, -1e30], np.float32)])
    got = grid_ref.e2m1_codes(torch.from_numpy(x)).numpy()
    np.testing.assert_array_equal(got, _e2m1_expected(x))


def _e4m3_expected(x: np.ndarray) -> np.ndarray:
    """RNE onto e4m3fn (bias 7, 3 mantissa bits, subnormal step 2^-9), |x| <= 448."""
    mags = []
    for e in range(16):
        for m in range(8):
            if e == 15 and m == 7:
                continue
            v = m * 2.0**-9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
            mags.append((v, (e << 3) | m))
    vals = np.array([v for v, _ in mags])
    codes = np.array([c for _, c in mags])
    ax = np.abs(x.astype(np.float64))
    i = np.searchsorted(vals, ax)  # vals[i-1] < ax <= vals[i]
    i = np.clip(i, 1, len(vals) - 1)
    lo, hi = vals[i - 1], vals[i]
    pick_hi = (ax - lo > hi - ax) | ((ax - lo == hi - ax) & (codes[i] % 2 == 0))
    c = np.where(pick_hi, codes[i], codes[i - 1])
    c = np.where(ax == 0, 0, c)
    sign = np.signbit(x).astype(np.int64) << 7
    return (c | sign).astype(np.uint8)


def test_oracle_e4m3_matches_closed_form():
    rng = np.random.default_rng(4)
    grid_pts = []
    for e in range(-10, 9):
        for m in range(16):
            grid_pts.append((1 + m / 16) * 2.0**e)  # includes all midpoints
    gp = np.array(grid_pts, dtype=np.float32)
    u = gp.view(np.uint32).astype(np.int64)
    near = np.concatenate([b + np.arange(-3, 4) for b in u]).astype(np.uint32).view(np.float32)
    x = np.concatenate([near, -near, (rng.standard_normal(50000) * 30).astype(np.float32), np.float32([0.0, -0.0, 448.0, -448.0])])
    x = np.clip(x, -448, 448).astype(np.float32)
    sc = torch.ones(x.shape[0])
    q, dq = grid_ref.quantize_mxfp_with_scale(torch.from_numpy(x).unsqueeze(-1), sc, "mxfp8")
    np.testing.assert_array_equal(q.squeeze(-1).numpy(), _e4m3_expected(x))


def test_pack_known_answer():
    words = packing_ref.pack_q(np.arange(16, dtype=np.uint8), 4)
    assert words.dtype == np.uint32 and words.tolist() == [0x76543210, 0xFEDCBA98]
    assert packing_ref.unpack_q(words, 4, 16).tolist() == list(range(16))
    with pytest.raises(AssertionError):
        packing_ref.pack_q(np.zeros(4, dtype=np.uint8), 4)


def test_pack_layouts_agree():
    q = torch.randint(0, 16, (5, 64), dtype=torch.uint8)
    words = packing_ref.pack_q(q.numpy(), 4)
    assert np.array_equal(words.view(np.uint8).reshape(5, 32), packing_ref.pack_nibbles(q).numpy())
    assert torch.equal(packing_ref.unpack_nibbles(packing_ref.pack_nibbles(q)), q)
    for bits in (2, 8):
        qq = np.random.default_rng(bits).integers(0, 2**bits, (3, 64)).astype(np.uint8)
        np.testing.assert_array_equal(packing_ref.unpack_q(packing_ref.pack_q(qq, bits), bits, 64), qq)


def test_oracle_hessian_close_to_fp64():
    g = torch.Generator().manual_seed(9)
    X = (torch.randn(20000, 256, generator=g) * torch.exp(torch.randn(256, generator=g))).to(torch.bfloat16)
    H = hessian_ref.stash_hessian([X[:7000], X[7000:]], 256, chunk_rows=4096)
    assert hessian_ref.rel_frobenius(H, hessian_ref.hessian_fp64(X)) < 1e-5


def test_oracle_hinv_invariants():
    g = torch.Generator().manual_seed(10)
    A = torch.randn(3, 64, 200, generator=g)
    H = A @ A.transpose(1, 2)
    U = gptq_ref.prepare_hinv(H.clone(), 0.01)
    assert torch.equal(U, U.triu())
    assert (U.diagonal(dim1=-2, dim2=-1) > 0).all()
    lam = 0.01 * H.diagonal(dim1=-2, dim2=-1).mean(-1)
    Hd = H.double() + lam.double()[:, None, None] * torch.eye(64, dtype=torch.float64)
    I = U.double().transpose(1, 2) @ U.double() @ Hd
    assert (I - torch.eye(64, dtype=torch.float64)).abs().max() < 1e-3
