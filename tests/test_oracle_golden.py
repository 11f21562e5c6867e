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
