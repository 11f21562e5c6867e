"""Pin the CPU oracle to the reference: bit-exact on the golden vectors.

tests/golden/solver_golden.* were written by the reference's own solver
(tests/golden/make_golden.py). The oracle must reproduce every output bit
for bit on this torch build, plus the in-place Hessian mutation, the damping
escalation warnings and the failure message.
"""

from __future__ import annotations

import logging

import pytest
import torch

from oracle import gptq_ref, grid_ref
from tests import golden_io


@pytest.fixture(scope="module")
def golden():
    return golden_io.load()


def _cases():
    _, meta = golden_io.load()
    return sorted(meta["cases"])


@pytest.mark.parametrize("name", _cases())
def test_oracle_solve_matches_reference_bits(golden, name):
    t, meta = golden
    kw = golden_io.case_kwargs(meta["cases"][name])
    W, H = t[f"{name}.W"].clone(), t[f"{name}.H"].clone()
    q, s, b, W_dq, rel = gptq_ref.solve_gptq(W, H, **kw)
    assert torch.equal(q, t[f"{name}.q"])
    assert torch.equal(s, t[f"{name}.scales"])
    if b is None:
        assert f"{name}.biases" not in t
    else:
        assert torch.equal(b, t[f"{name}.biases"])
    assert torch.equal(W_dq, t[f"{name}.W_dq"])
    assert torch.equal(rel, t[f"{name}.rel"])
    assert torch.equal(H, t[f"{name}.H_after"])  # dead-column diagonal written in place
    assert torch.equal(W, t[f"{name}.W"])  # solve_gptq leaves W_orig intact


def test_oracle_hinv_escalation_matches_reference(golden, caplog):
    t, meta = golden
    with caplog.at_level(logging.WARNING, logger="oracle.gptq_ref"):
        U = gptq_ref.prepare_hinv(t["hinv.H_ok"].clone(), 0.01)
    assert torch.equal(U, t["hinv.U_ok"])
    assert [r.getMessage() for r in caplog.records] == meta["hinv_ok_warnings"]
    caplog.clear()
    with caplog.at_level(logging.WARNING, logger="oracle.gptq_ref"):
        with pytest.raises(RuntimeError) as ei:
            gptq_ref.prepare_hinv(t["hinv.H_fail"].clone(), 0.01)
    assert str(ei.value) == meta["hinv_fail_message"]
    assert [r.getMessage() for r in caplog.records] == meta["hinv_fail_warnings"]


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("st", ["bfloat16", "float16", "float32"])
def test_oracle_choose_qparams_matches_reference(golden, bits, st):
    t, _ = golden
    dt = getattr(torch, st)
    _, _, s32, b32 = grid_ref.choose_qparams(t["qparams.w"], bits, "mse", dt)
    assert torch.equal(s32, t[f"qparams.b{bits}.{st}.s32"])
    assert torch.equal(b32, t[f"qparams.b{bits}.{st}.b32"])


@pytest.mark.parametrize("name", _cases())
def test_oracle_dequantize_artifact_matches_reference_w_dq(golden, name):
    """The reference's solver emits W_dq from the same codes and scales it
    returns (grid.py:108-124 and 215-221 inside gptq.py's loops), so its
    golden (q, scales, biases) triples pin the oracle's dequantize_artifact /
    dequantize_mxfp (grid.py:127-139, 154-164) bit for bit: E2M1 and E4M3
    decoding times 2^(byte-127) for the MXFP cases, q*s + b in fp32 for the
    affine ones."""
    t, meta = golden
    kw = golden_io.case_kwargs(meta["cases"][name])
    mode = kw.get("mode", "affine")
    G = kw["group_size"]
    q, s = t[f"{name}.q"], t[f"{name}.scales"]
    b = t.get(f"{name}.biases")
    dq = grid_ref.dequantize_artifact(q, s, b, mode, G)
    assert dq.dtype == torch.float32
    assert torch.equal(dq, t[f"{name}.W_dq"])
    if mode != "affine":
        dm = grid_ref.dequantize_mxfp(q, s, mode)
        assert torch.equal(dm.reshape(q.shape), t[f"{name}.W_dq"])
