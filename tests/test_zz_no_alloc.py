"""mgq_gptq_mxfp_noalloc (the solver on the library's fixed per-GPU scratch
array) against mgq_gptq_mxfp (the same solver on a caller workspace), both
called through the C ABI: every output bit for bit, on two calls in a row,
the second smaller than the first (the array keeps the first call's
contents), and an oversized request refused before anything is launched."""

from __future__ import annotations

import ctypes

import pytest
import torch

from mlx_gptq import _native as nat

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
OFFS = (0, -1, -2, -3, -4, 1, 2)


def _problem(B, R, C, seed):
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(B, R, C, generator=g) * 0.02).to(torch.bfloat16)
    X = torch.randn(B, 4 * C, C, generator=g) * torch.exp(torch.randn(C, generator=g))
    H = X.transpose(1, 2) @ X
    H[:, 5, :] = 0.0
    H[:, :, 5] = 0.0  # a dead column: its diagonal becomes 1 in place
    return W.to(DEV), H.contiguous().to(DEV)


def _outputs(B, R, C):
    return (torch.empty(B, R, C, dtype=torch.uint8, device=DEV),
            torch.empty(B, R, C // 32, dtype=torch.uint8, device=DEV),
            torch.empty(B, R, C, dtype=torch.float32, device=DEV),
            torch.empty(B, dtype=torch.float32, device=DEV),
            torch.empty(C // 32, B, dtype=torch.int32, device=DEV))


def _solve(entry, W, H, ws=None):
    lib = nat.load()
    B, R, C = W.shape
    q, s, W_dq, rel, att = _outputs(B, R, C)
    offs = (ctypes.c_int32 * len(OFFS))(*OFFS)
    args = [W.data_ptr(), nat.DTYPE_BF16, B, R, C, H.data_ptr(), nat.MODE_MXFP4, 1, 0.01, 6,
            ctypes.addressof(offs), len(OFFS), q.data_ptr(), s.data_ptr(), W_dq.data_ptr(),
            rel.data_ptr(), att.data_ptr()]
    if ws is not None:
        args += [ws.data_ptr(), ws.numel()]
    rc = getattr(lib, entry)(*args, nat.stream_of(DEV))
    assert rc == nat.OK, nat.last_error()
    torch.cuda.synchronize()
    return q, s, W_dq, rel, att, H


@pytest.mark.parametrize("shapes", [((24, 256, 512), (5, 64, 256))])
def test_noalloc_equals_workspace_entry_on_two_calls(shapes):
    lib = nat.load()
    for i, (B, R, C) in enumerate(shapes):
        W, H = _problem(B, R, C, seed=100 + i)
        ws = torch.empty(int(lib.mgq_gptq_mxfp_workspace_size(B, R, C)), dtype=torch.uint8,
                         device=DEV)
        want = _solve("mgq_gptq_mxfp", W, H.clone(), ws)
        got = _solve("mgq_gptq_mxfp_noalloc", W, H.clone())
        for a, b, name in zip(got, want, ("q", "scales", "W_dq", "rel_err", "attempts", "H")):
            assert torch.equal(a, b), (i, name)
        assert bool((got[4] == 1).all())  # every block factored at the first damping
        assert float(got[5][0, 5, 5]) == 1.0


def test_noalloc_refuses_more_than_its_scratch():
    lib = nat.load()
    cap = int(lib.mgq_noalloc_scratch_bytes())
    assert cap == 32 << 20
    B, R, C = 256, 2048, 2048  # needs ~140 MB: refused before any launch
    assert int(lib.mgq_gptq_mxfp_workspace_size(B, R, C)) > cap
    offs = (ctypes.c_int32 * len(OFFS))(*OFFS)
    rc = lib.mgq_gptq_mxfp_noalloc(None, nat.DTYPE_BF16, B, R, C, None, nat.MODE_MXFP4, 1, 0.01,
                                   6, ctypes.addressof(offs), len(OFFS), None, None, None, None,
                                   None, nat.stream_of(DEV))
    assert rc == nat.ERR_WORKSPACE
    assert "more than the" in nat.last_error() and "split the batch" in nat.last_error()
