"""The drop-in surface: every name the reference's Stage-A/B callers import
from the solver modules exists here with a compatible signature, and every
attribute they read on the capture manager, its stashes and tasks, and the
artifact writer and reader exists on this build's objects.

The expectations come from tests/golden/reference_api.json, written by
tests/golden/make_api_fixture.py from the reference sources parsed as text
(sequential.py, calibrate.py, dflash2_calibrate.py, pack.py, stream_pack.py,
validate_artifacts.py, qat.py, dflash2_distill.py). CPU only: nothing here
computes.
"""

from __future__ import annotations

import ast
import dataclasses
import importlib
import inspect
import json
import os
import subprocess
import sys
import textwrap
from pathlib import Path

import pytest
import torch

FIXTURE = Path(__file__).parent / "golden" / "reference_api.json"
API = json.loads(FIXTURE.read_text())
PKG = Path(__file__).resolve().parent.parent / "mlx-gptq-mxfp_amd"


def _value(src: str):
    """A reference default, from its source text (literals and torch.* names)."""
    node = ast.parse(src, mode="eval").body
    try:
        return ast.literal_eval(node)
    except ValueError:
        parts = []
        while isinstance(node, ast.Attribute):
            parts.append(node.attr)
            node = node.value
        assert isinstance(node, ast.Name) and node.id == "torch", src
        obj = torch
        for p in reversed(parts):
            obj = getattr(obj, p)
        return obj


_KINDS = {
    "positional": (inspect.Parameter.POSITIONAL_OR_KEYWORD, inspect.Parameter.POSITIONAL_ONLY),
    "keyword_only": (inspect.Parameter.KEYWORD_ONLY,),
    "var_positional": (inspect.Parameter.VAR_POSITIONAL,),
    "var_keyword": (inspect.Parameter.VAR_KEYWORD,),
}


def _check_params(where: str, ref: list[dict], fn) -> None:
    ours = list(inspect.signature(fn).parameters.values())
    if ref and ref[0]["name"] == "self":
        ref = ref[1:]
        ours = ours[1:]
    for i, rp in enumerate(ref):
        assert i < len(ours), f"{where}: missing parameter {rp['name']!r}"
        op = ours[i]
        assert op.name == rp["name"], f"{where}: parameter {i} is {op.name!r}, reference {rp['name']!r}"
        assert op.kind in _KINDS[rp["kind"]], f"{where}: {op.name} kind {op.kind}"
        if rp["default"] is not None:
            assert op.default is not inspect.Parameter.empty, f"{where}: {op.name} needs a default"
            assert op.default == _value(rp["default"]), \
                f"{where}: {op.name} default {op.default!r} != {rp['default']}"
    for extra in ours[len(ref):]:
        assert (extra.default is not inspect.Parameter.empty
                or extra.kind in (inspect.Parameter.VAR_POSITIONAL, inspect.Parameter.VAR_KEYWORD)), \
            f"{where}: extra parameter {extra.name!r} without a default"


def _ours(key: str):
    mod, name = key.split(".")
    return getattr(importlib.import_module(f"mlx_gptq.{mod}"), name)


@pytest.mark.parametrize("imp", API["imports"], ids=lambda i: f"{i['caller']}:{i['name']}")
def test_every_imported_name_exists(imp):
    mod = importlib.import_module(f"mlx_gptq.{imp['module']}")
    assert hasattr(mod, imp["name"]), f"{imp['caller']} imports {imp['module']}.{imp['name']}"


@pytest.mark.parametrize("key", sorted(API["defs"]))
def test_signatures_are_compatible(key):
    ref = API["defs"][key]
    obj = _ours(key)
    if ref["kind"] == "function":
        assert callable(obj), key
        _check_params(key, ref["params"], obj)
    elif ref["kind"] == "class":
        assert inspect.isclass(obj), key
        if ref["dataclass_fields"]:
            assert dataclasses.is_dataclass(obj), key
            assert [f.name for f in dataclasses.fields(obj)] == ref["dataclass_fields"], key
        for meth, spec in ref["methods"].items():
            if meth == "__init__" and ref["dataclass_fields"]:
                continue
            assert hasattr(obj, meth), f"{key}.{meth} missing"
            attr = inspect.getattr_static(obj, meth)
            if spec["property"]:
                assert isinstance(attr, property), f"{key}.{meth} should be a property"
            else:
                _check_params(f"{key}.{meth}", spec["params"], getattr(obj, meth))


def _toy_layer():
    transformers = pytest.importorskip("transformers")
    from transformers import Qwen3MoeConfig
    from transformers.models.qwen3_moe.modeling_qwen3_moe import Qwen3MoeSparseMoeBlock

    cfg = Qwen3MoeConfig(hidden_size=64, moe_intermediate_size=32, num_experts=4,
                         num_experts_per_tok=2)
    layer = torch.nn.Module()
    layer.self_attn = torch.nn.Module()
    layer.self_attn.q_proj = torch.nn.Linear(64, 64, bias=False)
    layer.mlp = Qwen3MoeSparseMoeBlock(cfg)
    return layer


def test_caller_attributes_exist(tmp_path):
    from mlx_gptq import capture
    from mlx_gptq.artifacts import ArtifactReader, ArtifactWriter

    mgr = capture.CaptureManager(_toy_layer(), None, 32)
    assert [t.name for t in mgr.linear_tasks] == ["self_attn.q_proj"]
    assert {(t.module_name, t.param_name) for t in mgr.fused_tasks} == {
        ("mlp.experts", "gate_up_proj"), ("mlp.experts", "down_proj")}
    w = ArtifactWriter(str(tmp_path), {"model": "toy", "mode": "mxfp8", "bits": 8,
                                       "group_size": 32, "storage_dtype": "bfloat16"})
    w.write_layer(0, {"a.weight": (torch.zeros(2, 32, dtype=torch.uint8),
                                   torch.full((2, 1), 127, dtype=torch.uint8), None)},
                  {"a.weight": {"bits": 8, "group_size": 32, "mode": "mxfp8"}})
    objects = {
        "CaptureManager": [mgr],
        "LinearTask": mgr.linear_tasks,
        "FusedExpertTask": mgr.fused_tasks,
        "Stash": [mgr.stashes["self_attn.q_proj"], mgr.stashes["mlp.experts.gate_up_proj::e0"],
                  mgr.stashes["mlp.experts.down_proj::e3"]],
        "ArtifactWriter": [w],
        "ArtifactReader": [ArtifactReader(str(tmp_path))],
    }
    for cls, attrs in API["uses"].items():
        for obj in objects[cls]:
            for a in attrs:
                assert hasattr(obj, a), f"{type(obj).__name__} lacks {a!r} (used on {cls})"


def test_expert_stash_keys_and_empty_views():
    from mlx_gptq import capture

    mgr = capture.CaptureManager(_toy_layer(), r"q_proj", 32)
    assert mgr.linear_tasks == []  # excluded by the regex
    (gu,) = [t for t in mgr.fused_tasks if t.param_name == "gate_up_proj"]
    assert gu.stash_keys == [f"mlp.experts.gate_up_proj::e{e}" for e in range(4)]
    assert gu.num_experts == 4 and gu.param.shape == (4, 64, 64)
    st = mgr.stashes[gu.stash_keys[1]]
    assert st.tokens == 0 and st.chunks == [] and st.nbytes() == 0
    assert mgr.expert_token_stats() == {"mlp.experts.gate_up_proj": (0, 0, 0, 4),
                                        "mlp.experts.down_proj": (0, 0, 0, 4)}
    with pytest.raises(RuntimeError, match="No tokens captured for fused experts"):
        mgr.check_capture_happened()


def test_reference_checkout_resolves_the_other_modules(tmp_path):
    """MLX_GPTQ_REFERENCE appends a checkout to the package path: modules
    missing here import from it, modules present here keep this build's."""
    ref = tmp_path / "checkout" / "mlx_gptq"
    ref.mkdir(parents=True)
    (ref / "__init__.py").write_text("")
    (ref / "sequential.py").write_text("from .capture import CaptureManager\nFROM = 'checkout'\n")
    (ref / "capture.py").write_text("raise ImportError('the checkout capture must not load')\n")
    code = textwrap.dedent("""
        import mlx_gptq.sequential as s, mlx_gptq.capture as c
        assert s.FROM == 'checkout'
        assert s.CaptureManager is c.CaptureManager
        assert 'mlx-gptq-mxfp_amd' in c.__file__
        print('ok')
    """)
    env = {**os.environ, "MLX_GPTQ_REFERENCE": str(tmp_path / "checkout"),
           "PYTHONPATH": str(PKG)}
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "ok"


def test_capture_manager_backfill_and_fallback_keys():
    """Never-routed experts are backfilled through the manager
    (capture.py:254-322) and reported under the reference's stash keys."""
    from mlx_gptq import capture

    layer = _toy_layer()
    blk = layer.mlp
    gate_fwd = blk.gate.forward

    def never_three(h):  # the router never picks expert 3
        logits, _, _ = gate_fwd(h)
        masked = logits.clone()
        masked[:, 3] = -float("inf")
        probs = torch.softmax(masked, dim=-1, dtype=torch.float)
        vals, idx = torch.topk(probs, 2, dim=-1)
        return logits, (vals / vals.sum(-1, keepdim=True)).to(logits.dtype), idx

    blk.gate.forward = never_three
    layer.forward = lambda x: blk(layer.self_attn.q_proj(x))
    mgr = capture.CaptureManager(layer, None, 32)
    g = torch.Generator().manual_seed(0)
    with torch.no_grad(), mgr:
        for _ in range(2):
            mgr.begin_batch()
            layer(torch.randn(1, 40, 64, generator=g))
    mgr.check_capture_happened()
    assert mgr.stashes["mlp.experts.gate_up_proj::e3"].tokens == 0
    zero = [e for e in range(4) if mgr.stashes[f"mlp.experts.gate_up_proj::e{e}"].tokens == 0]
    assert 3 in zero and mgr.expert_token_stats()["mlp.experts.gate_up_proj"][3] == len(zero)
    assert mgr.backfill_unrouted_experts() == {"mlp.experts": zero}
    assert mgr.fallback_experts == {f"mlp.experts.{p}::e{e}": "all_expert_inputs"
                                    for e in zero for p in ("gate_up_proj", "down_proj")}
    # the block's sampled inputs (64 evenly spaced rows of each 40-row batch: all of them)
    assert mgr.stashes["mlp.experts.gate_up_proj::e3"].tokens == 80
    assert mgr.stashes["mlp.experts.down_proj::e3"].tokens == 80
    assert mgr.stashes["self_attn.q_proj"].tokens == 80
    mgr.drop_all()
    assert mgr.total_stash_bytes() == 0
