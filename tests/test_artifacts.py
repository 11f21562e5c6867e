"""Artifact store (artifacts.ArtifactWriter / ArtifactReader) against the
reference's on-disk format (mlx_gptq/artifacts.py:1-139).

The format is checked from the outside: the manifest as plain JSON and the
layer files through safetensors, with the expected contents written out
here from the format description (tensor names ``{name}.q`` / ``.scales`` /
``.biases``, 4-bit codes nibble-packed low nibble first, ``q_packed``,
``has_biases``, ``file``, ``layers_done``). Files laid out that way by hand
must read back through ``ArtifactReader``, and the writer's files must hold
exactly that layout. The mxfp8 case follows the reference's own
test_mxfp_artifacts.py:16-72 (codes [3, 32], E8M0 scales [3, 1]).
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from safetensors.torch import load_file, save_file

from mlx_gptq.artifacts import ArtifactReader, ArtifactWriter

HEADER = {"model": "synthetic", "mode": "mxfp8", "bits": 8, "group_size": 32,
          "storage_dtype": "bfloat16"}


def _nibbles(q: np.ndarray) -> np.ndarray:
    return (q[..., 0::2] | (q[..., 1::2] << 4)).astype(np.uint8)


def test_raw_layer_round_trip_and_manifest(tmp_path):
    rng = np.random.default_rng(31)
    codes = rng.integers(0, 256, (3, 32), dtype=np.uint8)
    scales = rng.integers(110, 140, (3, 1), dtype=np.uint8)
    key = "model.layers.0.proj.weight"
    w = ArtifactWriter(str(tmp_path), dict(HEADER))
    meta = {key: {"mode": "mxfp8", "bits": 8, "group_size": 32, "kind": "linear"}}
    w.write_layer(0, {key: (torch.from_numpy(codes), torch.from_numpy(scales), None)}, meta)

    man = json.loads((tmp_path / "manifest.json").read_text())
    assert man == {**HEADER, "layers_done": [0], "tensors": {key: {
        "mode": "mxfp8", "bits": 8, "group_size": 32, "kind": "linear",
        "q_packed": "raw", "has_biases": False, "file": "layer_0000.safetensors"}}}
    blob = load_file(str(tmp_path / "layer_0000.safetensors"))
    assert sorted(blob) == [f"{key}.q", f"{key}.scales"]
    assert torch.equal(blob[f"{key}.q"], torch.from_numpy(codes))
    assert [p.name for p in tmp_path.iterdir() if p.name.endswith(".tmp")] == []

    r = ArtifactReader(str(tmp_path))
    q, s, b, info = r.get(key)
    assert torch.equal(q, torch.from_numpy(codes)) and torch.equal(s, torch.from_numpy(scales))
    assert b is None and info["has_biases"] is False
    assert r.has(key) and not r.has("x") and r.storage_dtype == torch.bfloat16


def test_resume_keeps_layers_and_rejects_mismatch(tmp_path):
    w = ArtifactWriter(str(tmp_path), dict(HEADER))
    meta = {"a": {"bits": 8}}
    w.write_layer(3, {"a": (torch.zeros(2, 32, dtype=torch.uint8), torch.ones(2, 1, dtype=torch.uint8),
                            None)}, meta)
    w2 = ArtifactWriter(str(tmp_path), dict(HEADER))
    assert w2.layer_done(3) and not w2.layer_done(0)
    with pytest.raises(RuntimeError, match="resume mismatch: manifest has bits=8, run has 4"):
        ArtifactWriter(str(tmp_path), {**HEADER, "bits": 4})
    ArtifactWriter(str(tmp_path), {**HEADER, "model": "other"})  # not a resume key


def test_reader_takes_a_hand_laid_raw_store(tmp_path):
    q = torch.arange(64, dtype=torch.uint8).reshape(2, 32)
    s = torch.tensor([[127], [130]], dtype=torch.uint8)
    save_file({"w.q": q, "w.scales": s}, str(tmp_path / "layer_0007.safetensors"))
    (tmp_path / "manifest.json").write_text(json.dumps({
        **HEADER, "layers_done": [7],
        "tensors": {"w": {"bits": 8, "q_packed": "raw", "has_biases": False,
                          "file": "layer_0007.safetensors"}}}))
    q2, s2, b2, _ = ArtifactReader(str(tmp_path)).get("w")
    assert torch.equal(q2, q) and torch.equal(s2, s) and b2 is None


@pytest.mark.gpu
def test_gpu_nibble_layer_from_device_tensors(tmp_path):
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(4)
    qa = torch.randint(0, 16, (64, 128), generator=g, dtype=torch.uint8)
    sa = torch.randn(64, 2, generator=g).to(torch.bfloat16)
    ba = torch.randn(64, 2, generator=g).to(torch.bfloat16)
    qm = torch.randint(0, 16, (3, 32, 64), generator=g, dtype=torch.uint8)
    sm = torch.randint(100, 140, (3, 32, 2), generator=g, dtype=torch.uint8)
    w = ArtifactWriter(str(tmp_path), {**HEADER, "mode": "mxfp4", "bits": 4})
    meta = {"aff": {"bits": 4, "mode": "affine"}, "mx": {"bits": 4, "mode": "mxfp4"}}
    w.write_layer(1, {"aff": (qa.to(dev), sa.to(dev), ba.to(dev)), "mx": (qm.to(dev), sm.to(dev), None)},
                  meta)
    blob = load_file(str(tmp_path / "layer_0001.safetensors"))
    assert sorted(blob) == ["aff.biases", "aff.q", "aff.scales", "mx.q", "mx.scales"]
    np.testing.assert_array_equal(blob["aff.q"].numpy(), _nibbles(qa.numpy()))
    np.testing.assert_array_equal(blob["mx.q"].numpy(), _nibbles(qm.numpy()))
    assert torch.equal(blob["aff.biases"], ba) and torch.equal(blob["mx.scales"], sm)
    man = json.loads((tmp_path / "manifest.json").read_text())
    assert man["tensors"]["aff"]["q_packed"] == "nibble" and man["tensors"]["aff"]["has_biases"] is True
    r = ArtifactReader(str(tmp_path))
    q, s, b, _ = r.get("aff")
    assert torch.equal(q, qa) and torch.equal(s, sa) and torch.equal(b, ba)
    q, s, b, _ = r.get("mx")
    assert torch.equal(q, qm) and torch.equal(s, sm) and b is None


@pytest.mark.gpu
def test_gpu_reader_takes_a_hand_laid_nibble_store(tmp_path):
    g = torch.Generator().manual_seed(6)
    q = torch.randint(0, 16, (5, 96), generator=g, dtype=torch.uint8)
    save_file({"n.q": torch.from_numpy(_nibbles(q.numpy())), "n.scales": torch.ones(5, 3)},
              str(tmp_path / "layer_0000.safetensors"))
    (tmp_path / "manifest.json").write_text(json.dumps({
        **HEADER, "layers_done": [0],
        "tensors": {"n": {"bits": 4, "q_packed": "nibble", "has_biases": False,
                          "file": "layer_0000.safetensors"}}}))
    q2, _, _, _ = ArtifactReader(str(tmp_path)).get("n")
    assert torch.equal(q2, q)
