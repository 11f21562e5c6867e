"""Artifact range audit: the oracle (oracle/validate_ref.py, a restatement
of validate_artifacts.py:15-55) pinned on closed-form cases, then the fused
device pass (validate_artifacts.range_audit -> mgq_range_audit) against it,
and the report of validate() over an artifact store."""

from __future__ import annotations

import math

import pytest
import torch

from mlx_gptq import validate_artifacts as va
from oracle import grid_ref, validate_ref


def _mx(rows, groups, code, byte):
    q = torch.full((rows, 32 * groups), code, dtype=torch.uint8)
    s = torch.full((rows, groups), byte, dtype=torch.uint8)
    return q, s


def test_oracle_closed_forms():
    src = torch.ones(2, 64)
    # E2M1 code 2 is 1.0, byte 127 is 2^0: deq == source, ratio 1 / 32
    q, s = _mx(2, 2, 2, 127)
    st = validate_ref.range_audit(src, q, s, None, "mxfp4", 32)
    assert st == {"nonfinite": 0, "exceed": 0, "ratio": 1 / 32, "source_max": 1.0, "artifact_max": 1.0}
    # code 7 (6.0) at 2^6: 384 against a limit of 32
    q, s = _mx(2, 2, 7, 133)
    st = validate_ref.range_audit(src, q, s, None, "mxfp4", 32)
    assert st["exceed"] == 4 and st["ratio"] == 12.0 and st["artifact_max"] == 384.0
    # all-zero source: the limit is 2^-126
    q, s = _mx(1, 1, 1, 127)  # 0.5
    st = validate_ref.range_audit(torch.zeros(1, 32), q, s, None, "mxfp4", 32)
    assert st["exceed"] == 1 and st["ratio"] == 0.5 * 2.0**126
    q, s = _mx(1, 1, 0, 127)
    assert validate_ref.range_audit(torch.zeros(1, 32), q, s, None, "mxfp4", 32)["ratio"] == 0.0
    # byte 255 is 2^128 = inf in fp32: code 0 gives NaN, others inf
    q, s = _mx(1, 1, 0, 255)
    q[0, 5] = 3
    assert validate_ref.range_audit(torch.ones(1, 32), q, s, None, "mxfp4", 32)["nonfinite"] == 32
    # affine: q * s + b = 4 * 0.5 - 1 = 1 against a source of 1
    q = torch.full((3, 128), 4, dtype=torch.uint8)
    sc = torch.full((3, 2), 0.5, dtype=torch.bfloat16)
    b = torch.full((3, 2), -1.0, dtype=torch.bfloat16)
    st = validate_ref.range_audit(torch.ones(3, 128), q, sc, b, "affine", 64)
    assert st["ratio"] == 1 / 32 and st["exceed"] == 0
    # mxfp8: E4M3 0x38 is 1.0, 0x7e is 448
    q, s = _mx(1, 1, 0x7E, 127)
    st = validate_ref.range_audit(torch.full((1, 32), 2.0), q, s, None, "mxfp8", 32)
    assert st["ratio"] == 448 / 64 and st["exceed"] == 1


def test_validation_errors():
    with pytest.raises(ValueError):
        va.range_audit(torch.ones(2, 32), torch.zeros(2, 32, dtype=torch.uint8),
                       torch.zeros(2, 1, dtype=torch.uint8), None, "int4", 32)
    with pytest.raises(ValueError):
        va.range_audit(torch.ones(2, 48), torch.zeros(2, 48, dtype=torch.uint8),
                       torch.zeros(2, 1, dtype=torch.uint8), None, "mxfp4", 32)
    with pytest.raises(ValueError):
        va.range_audit(torch.ones(2, 32), torch.zeros(3, 32, dtype=torch.uint8),
                       torch.zeros(2, 1, dtype=torch.uint8), None, "mxfp4", 32)


def _random_case(mode, rows, cols, seed, src_dtype=torch.bfloat16, gs=64):
    g = torch.Generator().manual_seed(seed)
    src = (torch.randn(rows, cols, generator=g) * torch.exp(torch.randn(rows, 1, generator=g))).to(src_dtype)
    if mode == "affine":
        q = torch.randint(0, 16, (rows, cols), generator=g, dtype=torch.uint8)
        s = (torch.rand(rows, cols // gs, generator=g) * 0.2).to(torch.bfloat16)
        b = (torch.randn(rows, cols // gs, generator=g) * 0.5).to(torch.bfloat16)
        return src, q, s, b, gs
    q, s, _, _ = grid_ref.rtn_quantize_mxfp(src.float(), mode)
    # perturb some groups past the limit
    s = s.clone()
    s.view(-1)[:: 7] += 6
    return src, q, s, None, 32


@pytest.mark.gpu
@pytest.mark.parametrize("mode,rows,cols,seed", [("mxfp4", 96, 256, 1), ("mxfp8", 33, 2048, 2),
                                                 ("affine", 50, 512, 3), ("mxfp4", 1, 32, 4),
                                                 ("mxfp4", 777, 4096, 5)])
def test_gpu_range_audit_matches_oracle(mode, rows, cols, seed):
    src, q, s, b, gs = _random_case(mode, rows, cols, seed)
    want = validate_ref.range_audit(src, q, s, b, mode, gs)
    dev = torch.device("cuda", 0)
    got = va.range_audit(src.to(dev), q.to(dev), s.to(dev), None if b is None else b.to(dev), mode, gs)
    assert got == want


@pytest.mark.gpu
def test_gpu_range_audit_closed_forms_and_nonfinite():
    dev = torch.device("cuda", 0)
    q, s = _mx(1, 1, 0, 255)
    q[0, 5] = 3
    st = va.range_audit(torch.ones(1, 32, device=dev), q.to(dev), s.to(dev), None, "mxfp4", 32)
    assert st["nonfinite"] == 32
    q, s = _mx(1, 1, 1, 127)
    st = va.range_audit(torch.zeros(1, 32, device=dev), q.to(dev), s.to(dev), None, "mxfp4", 32)
    assert st["exceed"] == 1 and st["ratio"] == 0.5 * 2.0**126
    src = torch.ones(2, 64, dtype=torch.float16, device=dev)
    q, s = _mx(2, 2, 2, 127)
    st = va.range_audit(src, q.to(dev), s.to(dev), None, "mxfp4", 32)
    assert st == {"nonfinite": 0, "exceed": 0, "ratio": 1 / 32, "source_max": 1.0, "artifact_max": 1.0}


@pytest.mark.gpu
def test_gpu_validate_report(tmp_path):
    from mlx_gptq.artifacts import ArtifactReader, ArtifactWriter

    dev = torch.device("cuda", 0)
    w = ArtifactWriter(str(tmp_path), {"mode": "mxfp4", "bits": 4, "group_size": 32,
                                       "storage_dtype": "bfloat16"})
    good = _random_case("mxfp4", 16, 128, 7)
    src_good = good[0]
    q_good, s_good, _, _ = grid_ref.rtn_quantize_mxfp(src_good.float(), "mxfp4")
    bad_q, bad_s = _mx(4, 2, 7, 140)
    tensors = {
        "a.good": (q_good.to(dev), s_good.to(dev), None),
        "b.bad": (bad_q.to(dev), bad_s.to(dev), None),
        "c.nan": (_mx(4, 1, 0, 255)[0].to(dev), _mx(4, 1, 0, 255)[1].to(dev), None),
        "d.shape": (torch.zeros(4, 32, dtype=torch.uint8, device=dev),
                    torch.full((4, 1), 127, dtype=torch.uint8, device=dev), None),
        "e.missing": (torch.zeros(2, 32, dtype=torch.uint8, device=dev),
                      torch.full((2, 1), 127, dtype=torch.uint8, device=dev), None),
    }
    meta = {k: {"bits": 4, "mode": "mxfp4", "group_size": 32} for k in tensors}
    w.write_layer(0, tensors, meta)
    sources = {"a.good": src_good, "b.bad": torch.ones(4, 64), "c.nan": torch.ones(4, 32),
               "d.shape": torch.ones(4, 64)}
    rep = va.validate(ArtifactReader(str(tmp_path)), sources, "m", "c")
    errs = {f["name"]: f["error"] for f in rep["failures"]}
    want_bad = validate_ref.range_audit(sources["b.bad"], bad_q, bad_s, None, "mxfp4", 32)
    assert errs == {"b.bad": f"group range ratio {want_bad['ratio']:.6g}",
                    "c.nan": "non-finite dequantized values",
                    "d.shape": "shape (4, 64) != (4, 32)",
                    "e.missing": "missing source tensor"}
    assert rep["status"] == "failed" and rep["tensors"] == 5
    assert [x["name"] for x in rep["worst"]] == ["b.bad", "a.good"]
    want_good = validate_ref.range_audit(src_good, q_good, s_good, None, "mxfp4", 32)
    assert rep["worst"][1]["ratio"] == round(want_good["ratio"], 6)
    assert math.isclose(rep["worst"][0]["artifact_max"], 6.0 * 2.0**13)
