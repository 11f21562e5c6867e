"""HIP Hessian (bf16 MFMA SYRK) vs the CPU oracle and float64.

Gate: H within 1e-5 relative Frobenius error of a
float64 X^T X of the same bf16 rows. Also: exact symmetry, the grouped and
gathered (routed expert) forms, empty groups (H = 0), accumulate mode, the
K-split partial-tile path, ragged token counts and channel counts that are
not tile multiples, and the Stash API.
"""

from __future__ import annotations

import pytest
import torch

from oracle import hessian_ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
TOL = 1e-5


def _rows(n, c, seed, outliers=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, c, generator=g) * torch.exp(torch.randn(c, generator=g))
    if outliers:
        idx = torch.randperm(c, generator=g)[:outliers]
        x[:, idx] *= 20.0
    return x.to(torch.bfloat16)


@pytest.mark.parametrize("n,c", [(5000, 96), (4099, 256), (8192, 768), (3000, 520), (64, 64)])
def test_dense_hessian_vs_fp64(n, c):
    from mlx_gptq import capture

    X = _rows(n, c, seed=n + c, outliers=max(1, c // 100))
    H = capture.hessian_xtx(X.to(DEV)).cpu()
    ref64 = hessian_ref.hessian_fp64(X)
    assert hessian_ref.rel_frobenius(H, ref64) < TOL
    assert torch.equal(H, H.T)
    # the reference's own fp32 path lands in the same place
    H_ref = hessian_ref.stash_hessian([X], c)
    assert hessian_ref.rel_frobenius(H_ref, ref64) < TOL


def test_grouped_gathered_hessian():
    from mlx_gptq import capture

    C, N = 256, 6000
    X = _rows(N, C, seed=3)
    g = torch.Generator().manual_seed(4)
    sizes = [700, 0, 1500, 33, 2048, 1]
    idx = torch.cat([torch.randint(0, N, (s,), generator=g) for s in sizes]).to(torch.int32)
    off = [0]
    for s in sizes:
        off.append(off[-1] + s)
    H = capture.grouped_hessian(X.to(DEV), off, row_index=idx.to(DEV)).cpu()
    assert H.shape == (len(sizes), C, C)
    for gi, s in enumerate(sizes):
        rows = X[idx[off[gi] : off[gi + 1]].long()]
        if s == 0:
            assert torch.count_nonzero(H[gi]) == 0
            continue
        assert hessian_ref.rel_frobenius(H[gi], hessian_ref.hessian_fp64(rows)) < TOL
        assert torch.equal(H[gi], H[gi].T)


def test_gathered_hessian_wide_addressing(monkeypatch):
    """The 64-bit per-token row addressing used when X spans more than 4 GB,
    forced on a small X: same H as the 32-bit row-offset form, bit for bit."""
    from mlx_gptq import capture

    C, N = 512, 3000
    X = _rows(N, C, seed=8).to(DEV)
    g = torch.Generator().manual_seed(9)
    sizes = [900, 0, 1300, 77]
    idx = torch.cat([torch.randint(0, N, (s,), generator=g) for s in sizes]).to(torch.int32)
    off = [0]
    for s in sizes:
        off.append(off[-1] + s)
    H32 = capture.grouped_hessian(X, off, row_index=idx.to(DEV))
    monkeypatch.setenv("MGQ_HESSIAN_WIDE_ADDR", "1")
    H64 = capture.grouped_hessian(X, off, row_index=idx.to(DEV))
    assert torch.equal(H32, H64)
    Xc = X.cpu()
    for gi, s in enumerate(sizes):
        if s:
            rows = Xc[idx[off[gi] : off[gi + 1]].long()]
            assert hessian_ref.rel_frobenius(H64[gi].cpu(), hessian_ref.hessian_fp64(rows)) < TOL


@pytest.mark.parametrize("c", [1, 13, 100, 2051])
def test_channel_counts_not_multiple_of_8(c):
    """Any C (the reference's Stash.hessian takes any width): dense, grouped
    and gathered, and accumulation into a caller's H, against float64; also
    rows that are not 16-byte aligned (a column slice of a wider matrix)."""
    from mlx_gptq import capture

    N = 3000
    X = _rows(N, c, seed=c)
    H = capture.hessian_xtx(X.to(DEV)).cpu()
    assert H.shape == (c, c) and torch.equal(H, H.T)
    assert hessian_ref.rel_frobenius(H, hessian_ref.hessian_fp64(X)) < TOL
    g = torch.Generator().manual_seed(c)
    sizes = [700, 0, 1800]
    idx = torch.cat([torch.randint(0, N, (k,), generator=g) for k in sizes]).to(torch.int32)
    off = [0, 700, 700, 2500]
    out = torch.zeros(3, c, c, device=DEV)
    capture.grouped_hessian(X.to(DEV), off, row_index=idx.to(DEV), out=out)
    capture.grouped_hessian(X.to(DEV), off, row_index=idx.to(DEV), out=out, accumulate=True)
    Hg = out.cpu()
    for gi in range(3):
        rows = X[idx[off[gi] : off[gi + 1]].long()]
        if rows.shape[0] == 0:
            assert torch.count_nonzero(Hg[gi]) == 0
            continue
        assert hessian_ref.rel_frobenius(Hg[gi], 2 * hessian_ref.hessian_fp64(rows)) < TOL
    wide = _rows(N, c + 3, seed=c + 1).to(DEV)
    Hs = capture.hessian_xtx(wide[:, 3:]).cpu()  # rows offset by 6 bytes
    assert hessian_ref.rel_frobenius(Hs, hessian_ref.hessian_fp64(wide[:, 3:].cpu())) < TOL


@pytest.mark.parametrize("C", [768, 1000])
def test_heavy_groups_split_and_diagonal_pairs(C):
    """A multi-group gathered launch in which the heaviest groups are split
    along K (partial tiles, summed by the reduce kernel) while the others run
    whole with their diagonal tiles in pairs (C = 768: one pair and one odd
    tile; C = 1000: two pairs, the last tile ragged). Every group against
    float64, exact symmetry, and accumulation onto the first result."""
    from mlx_gptq import capture

    N = 12000
    X = _rows(N, C, seed=C)
    g = torch.Generator().manual_seed(C + 1)
    sizes = [300, 9000, 0, 5000, 120]
    idx = torch.cat([torch.randint(0, N, (s,), generator=g) for s in sizes]).to(torch.int32)
    off = [0]
    for s in sizes:
        off.append(off[-1] + s)
    Xd, idd = X.to(DEV), idx.to(DEV)
    H = capture.grouped_hessian(Xd, off, row_index=idd)
    Hc = H.cpu()
    for gi, s in enumerate(sizes):
        if s == 0:
            assert torch.count_nonzero(Hc[gi]) == 0
            continue
        rows = X[idx[off[gi] : off[gi + 1]].long()]
        assert hessian_ref.rel_frobenius(Hc[gi], hessian_ref.hessian_fp64(rows)) < TOL
        assert torch.equal(Hc[gi], Hc[gi].T)
    out = H.clone()
    capture.grouped_hessian(Xd, off, row_index=idd, out=out, accumulate=True)
    assert torch.equal(out.cpu(), 2 * Hc)  # the same launch again, added exactly


def test_split_k_partials_and_accumulate():
    from mlx_gptq import capture

    C, N = 256, 20000  # one tile: the planner splits K into partial tiles
    X = _rows(N, C, seed=5)
    Xd = X.to(DEV)
    H = capture.grouped_hessian(Xd, [0, N], target_items=64).cpu()[0]
    ref64 = hessian_ref.hessian_fp64(X)
    assert hessian_ref.rel_frobenius(H, ref64) < TOL
    H2 = capture.grouped_hessian(Xd, [0, N], target_items=1).cpu()[0]  # no split
    assert hessian_ref.rel_frobenius(H2, ref64) < TOL
    out = torch.full((1, C, C), 0.0, device=DEV)
    capture.grouped_hessian(Xd[:12000], [0, 12000], out=out)
    capture.grouped_hessian(Xd[12000:], [0, N - 12000], out=out, accumulate=True)
    assert hessian_ref.rel_frobenius(out.cpu()[0], ref64) < TOL


def test_stash_api_matches_reference_semantics():
    from mlx_gptq import capture

    C = 128
    st = capture.Stash("layer.mlp", C)
    parts = [torch.randn(300, C), torch.randn(2, 5, C) * 3, torch.randn(1000, C)]
    for p in parts:
        st.add(p.to(DEV))
    assert st.tokens == 1310 and st.nbytes() == 1310 * C * 2
    H = st.hessian(DEV, chunk_rows=512).cpu()
    rows = [p.reshape(-1, C).to(torch.bfloat16) for p in parts]
    ref = hessian_ref.stash_hessian(rows, C, chunk_rows=512)
    assert hessian_ref.rel_frobenius(H, hessian_ref.hessian_fp64(torch.cat(rows))) < TOL
    assert hessian_ref.rel_frobenius(H, ref) < TOL
    with pytest.raises(RuntimeError):
        st.add(torch.randn(3, C + 1))
    st.clear()
    assert st.chunks == []


def test_moe_shaped_grouped_hessian_property():
    """Config-4 shape (C=2048, 32 experts of a routed batch): every expert's H
    against float64 on a sample of experts; exact symmetry for all."""
    from mlx_gptq import capture

    C, N, E = 2048, 16384, 32
    X = _rows(N, C, seed=6, outliers=20)
    g = torch.Generator().manual_seed(7)
    counts = torch.randint(0, 1200, (E,), generator=g)
    counts[3] = 0
    idx = torch.cat([torch.randperm(N, generator=g)[: int(c)] for c in counts]).to(torch.int32)
    off = [0] + torch.cumsum(counts, 0).tolist()
    H = capture.grouped_hessian(X.to(DEV), off, row_index=idx.to(DEV))
    assert torch.equal(H, H.transpose(1, 2))
    Hc = H.cpu()
    assert torch.count_nonzero(Hc[3]) == 0
    for e in (0, 5, 17, 31):
        rows = X[idx[off[e] : off[e + 1]].long()]
        assert hessian_ref.rel_frobenius(Hc[e], hessian_ref.hessian_fp64(rows)) < TOL
