"""Stage-B emission (pack.inject, pack.ShardEmitter) against the reference's
behaviour: the injection round trip of the reference's own
tests/test_mxfp_artifacts.py:16-72 (packed words equal ``pack_q`` of the
codes, scales carried over, no biases), switch_mlp stacking of per-expert
artifacts, affine biases, the RTN fallback, and the errors of
pack.py:90-227. Expected words come from the oracle (oracle/packing_ref.py,
pinned on the reference's known answers); shards are written and read with
safetensors and ``"format": "mlx"`` metadata, as mlx.save_safetensors does."""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import load_file, save_file

from mlx_gptq import pack
from mlx_gptq.artifacts import ArtifactReader, ArtifactWriter
from oracle import grid_ref, packing_ref


def _model(path, tensors, quant):
    path.mkdir(exist_ok=True)
    (path / "config.json").write_text(json.dumps({"quantization": quant}))
    save_file(tensors, str(path / "model.safetensors"), metadata={"format": "mlx"})


def _calib(path, mode, bits, tensors, group_size=32):
    w = ArtifactWriter(str(path), {"model": "synthetic", "mode": mode, "bits": bits,
                                   "group_size": group_size, "storage_dtype": "bfloat16"})
    meta = {k: {"mode": mode, "bits": bits, "group_size": group_size, "kind": "linear"} for k in tensors}
    w.write_layer(0, tensors, meta)
    return ArtifactReader(str(path))


def test_predicate_and_overrides(tmp_path):
    predicate = pack.make_predicate("", None, None, 32, mode="mxfp4")
    assert predicate("model.embed_tokens", object()) is False
    assert predicate("lm_head", object()) is False
    assert predicate("model.layers.0.mlp.down_proj", object()) is True
    p = pack.make_predicate(pack.ROUTER_SKIP, 8, None, 32, mode="mxfp4", path_bits={"a.b": 8})
    assert p("model.layers.0.mlp.gate", None) is False
    assert p("a.b", None) == {"group_size": 32, "bits": 8, "mode": "mxfp4"}
    assert p("lm_head", None) == {"group_size": 32, "bits": 8, "mode": "mxfp4"}
    (tmp_path / "manifest.json").write_text(json.dumps({"bits": 4, "layers_done": [], "tensors": {
        "m.layers.0.mlp.experts.3.down_proj.weight": {"bits": 8},
        "m.layers.0.mlp.experts.5.down_proj.weight": {"bits": 8},
        "m.layers.0.attn.q_proj.weight": {"bits": 4}}}))
    r = ArtifactReader(str(tmp_path))
    assert pack.overrides_from_manifest(r) == {"m.layers.0.mlp.switch_mlp.down_proj": 8}
    r.tensors["m.layers.0.mlp.experts.6.down_proj.weight"] = {"bits": 2}
    with pytest.raises(RuntimeError, match="conflicting expert bits"):
        pack.overrides_from_manifest(r)


@pytest.mark.gpu
@pytest.mark.parametrize("mode,bits", [("mxfp4", 4), ("mxfp8", 8)])
def test_gpu_native_mxfp_artifact_injection(tmp_path, mode, bits):
    key = "model.layers.0.proj.weight"
    base = key.removesuffix(".weight")
    rng = np.random.default_rng(31)
    codes = rng.integers(0, 2**bits, (3, 32), dtype=np.uint8)
    scales = rng.integers(110, 140, (3, 1), dtype=np.uint8)
    reader = _calib(tmp_path / "calibration", mode, bits,
                    {key: (torch.from_numpy(codes), torch.from_numpy(scales), None)})
    _model(tmp_path / "model", {key: torch.zeros(3, 32 * bits // 32, dtype=torch.uint32),
                                f"{base}.scales": torch.zeros(3, 1, dtype=torch.uint8)},
           {"mode": mode, "bits": bits, "group_size": 32})
    injected, kept = pack.inject(str(tmp_path / "model"), reader)
    assert injected == [key] and kept == []
    out = load_file(str(tmp_path / "model" / "model.safetensors"))
    np.testing.assert_array_equal(out[key].numpy(), packing_ref.pack_q(codes, bits))
    np.testing.assert_array_equal(out[f"{base}.scales"].numpy(), scales)
    assert f"{base}.biases" not in out
    with safe_open(str(tmp_path / "model" / "model.safetensors"), "pt") as f:
        assert f.metadata() == {"format": "mlx"}


@pytest.mark.gpu
def test_gpu_switch_mlp_stacking_affine_and_rtn_kept(tmp_path):
    E, R, C = 3, 8, 128
    g = torch.Generator().manual_seed(2)
    sw = "model.layers.0.mlp.switch_mlp.gate_proj.weight"
    arts, codes = {}, []
    for e in range(E):
        q = torch.randint(0, 16, (R, C), generator=g, dtype=torch.uint8)
        codes.append(q.numpy())
        arts[f"model.layers.0.mlp.experts.{e}.gate_proj.weight"] = (
            q, torch.randint(100, 140, (R, C // 32), generator=g, dtype=torch.uint8), None)
    reader = _calib(tmp_path / "c", "mxfp4", 4, arts)
    _model(tmp_path / "m", {
        sw: torch.zeros(E, R, C // 8, dtype=torch.uint32),
        sw.replace(".weight", ".scales"): torch.zeros(E, R, C // 32, dtype=torch.uint8),
        "model.layers.0.mlp.switch_mlp.up_proj.weight": torch.zeros(E, R, C // 8, dtype=torch.uint32),
        "model.layers.0.mlp.switch_mlp.up_proj.scales": torch.zeros(E, R, C // 32, dtype=torch.uint8),
        "model.embed_tokens.weight": torch.ones(4, 4),
    }, {"mode": "mxfp4", "bits": 4, "group_size": 32})
    injected, kept = pack.inject(str(tmp_path / "m"), reader)
    assert injected == [sw] and kept == ["model.layers.0.mlp.switch_mlp.up_proj.weight"]
    out = load_file(str(tmp_path / "m" / "model.safetensors"))
    np.testing.assert_array_equal(out[sw].numpy(), packing_ref.pack_q(np.stack(codes), 4))
    np.testing.assert_array_equal(out[sw.replace(".weight", ".scales")].numpy(),
                                  np.stack([a[1].numpy() for a in arts.values()]))
    assert torch.equal(out["model.embed_tokens.weight"], torch.ones(4, 4))

    # affine: biases carried in the shard's scale dtype
    key = "model.layers.1.o_proj.weight"
    q = torch.randint(0, 16, (4, 128), generator=g, dtype=torch.uint8)
    s = torch.rand(4, 2, generator=g).to(torch.bfloat16)
    b = torch.randn(4, 2, generator=g).to(torch.bfloat16)
    reader = _calib(tmp_path / "c2", "affine", 4, {key: (q, s, b)}, group_size=64)
    _model(tmp_path / "m2", {key: torch.zeros(4, 16, dtype=torch.uint32),
                             "model.layers.1.o_proj.scales": torch.zeros(4, 2, dtype=torch.bfloat16),
                             "model.layers.1.o_proj.biases": torch.zeros(4, 2, dtype=torch.bfloat16)},
           {"mode": "affine", "bits": 4, "group_size": 64})
    pack.inject(str(tmp_path / "m2"), reader)
    out = load_file(str(tmp_path / "m2" / "model.safetensors"))
    np.testing.assert_array_equal(out[key].numpy(), packing_ref.pack_q(q.numpy(), 4))
    assert torch.equal(out["model.layers.1.o_proj.biases"], b)
    assert torch.equal(out["model.layers.1.o_proj.scales"], s)


@pytest.mark.gpu
def test_gpu_inject_errors(tmp_path):
    g = torch.Generator().manual_seed(3)
    q = torch.randint(0, 16, (2, 32), generator=g, dtype=torch.uint8)
    s = torch.full((2, 1), 127, dtype=torch.uint8)
    sw = "model.layers.0.mlp.switch_mlp.down_proj.weight"
    reader = _calib(tmp_path / "c", "mxfp4", 4,
                    {"model.layers.0.mlp.experts.0.down_proj.weight": (q, s, None)})
    _model(tmp_path / "m", {sw: torch.zeros(2, 2, 4, dtype=torch.uint32),
                            sw.replace(".weight", ".scales"): torch.zeros(2, 2, 1, dtype=torch.uint8)},
           {"mode": "mxfp4", "bits": 4, "group_size": 32})
    with pytest.raises(RuntimeError, match="only some experts have artifacts"):
        pack.inject(str(tmp_path / "m"), reader)
    key = "model.layers.0.proj.weight"
    reader = _calib(tmp_path / "c2", "mxfp4", 4, {key: (q, s, None), "extra.weight": (q, s, None)})
    _model(tmp_path / "m2", {key: torch.zeros(2, 4, dtype=torch.uint32),
                             "model.layers.0.proj.scales": torch.zeros(2, 1, dtype=torch.uint8)},
           {"mode": "mxfp8", "bits": 8, "group_size": 32})
    # a dense tensor's mismatch uses the reference's short form (pack.py:163-173)
    with pytest.raises(RuntimeError, match="artifact mxfp4/4b/g32 vs config mxfp8/8b/g32"):
        pack.inject(str(tmp_path / "m2"), reader)
    _model(tmp_path / "m3", {key: torch.zeros(2, 4, dtype=torch.uint32),
                             "model.layers.0.proj.scales": torch.zeros(2, 1, dtype=torch.uint8)},
           {"mode": "mxfp4", "bits": 4, "group_size": 32})
    with pytest.raises(RuntimeError, match="never consumed"):
        pack.inject(str(tmp_path / "m3"), reader)


@pytest.mark.gpu
def test_gpu_shard_emitter(tmp_path):
    g = torch.Generator().manual_seed(4)
    E, R, C = 2, 4, 64
    arts = {f"model.layers.0.mlp.experts.{e}.up_proj.weight":
            (torch.randint(0, 16, (R, C), generator=g, dtype=torch.uint8),
             torch.randint(110, 130, (R, C // 32), generator=g, dtype=torch.uint8), None)
            for e in range(E)}
    arts["model.layers.0.attn.q_proj.weight"] = (torch.randint(0, 16, (R, C), generator=g, dtype=torch.uint8),
                                                 torch.full((R, 2), 125, dtype=torch.uint8), None)
    reader = _calib(tmp_path / "c", "mxfp4", 4, arts)
    em = pack.ShardEmitter(reader, "mxfp4", 4, 32)
    out = em.emit("model.layers.0.mlp.switch_mlp.up_proj.weight", torch.zeros(E, R, C))
    want = packing_ref.pack_q(np.stack([arts[f"model.layers.0.mlp.experts.{e}.up_proj.weight"][0].numpy()
                                        for e in range(E)]), 4)
    np.testing.assert_array_equal(out["model.layers.0.mlp.switch_mlp.up_proj.weight"], want)
    out = em.emit("model.layers.0.attn.q_proj.weight", torch.zeros(R, C))
    np.testing.assert_array_equal(out["model.layers.0.attn.q_proj.weight"],
                                  packing_ref.pack_q(arts["model.layers.0.attn.q_proj.weight"][0].numpy(), 4))
    W = torch.randn(R, C, generator=g).to(torch.bfloat16)
    out = em.emit("model.layers.0.attn.k_proj.weight", W)  # no artifact: RTN
    rq, rs, _, _ = grid_ref.rtn_quantize_mxfp(W.float().unsqueeze(0), "mxfp4")
    np.testing.assert_array_equal(out["model.layers.0.attn.k_proj.weight"], packing_ref.pack_q(rq[0].numpy(), 4))
    np.testing.assert_array_equal(out["model.layers.0.attn.k_proj.scales"], rs[0].numpy())
    assert set(em.emit("lm_head.weight", W)) == {"lm_head.weight"}
    assert em.stats == {"injected": E + 1, "rtn": 1, "kept": 1}
