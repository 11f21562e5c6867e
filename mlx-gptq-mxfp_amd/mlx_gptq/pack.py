"""Stage-B shard emission: calibrated artifacts into MLX-layout shards
(pack.py:33-227 and stream_pack.py:139-221 of the reference), with the
code packing and the RTN fallback on the HIP device.

``inject(mlx_path, reader)`` rewrites the shards of a converted MLX model
(``model*.safetensors`` with ``"format": "mlx"`` metadata plus
``config.json``'s ``quantization``) exactly as the reference does: every
quantized ``{base}.weight`` that has an artifact gets the artifact's codes
packed into uint32 words (``pack_q``), its scales cast to the shard's scale
dtype, and for affine its biases; a fused ``switch_mlp`` /
``experts.switch_glu`` tensor [E, out, words] takes the E per-expert
artifacts, stacked on the device and packed in one launch. Shards are read
and written with safetensors (no MLX runtime needed), each rewritten under a
temporary name and renamed. The same checks raise the same errors: a
mode/bits/group mismatch, experts with only some artifacts, packed or scale
shapes that differ from the converted model, affine without biases, and
artifacts never consumed.

``ShardEmitter.emit`` is the streaming packer's per-tensor rule
(stream_pack.py:155-221): stacked experts, one artifact, or MXFP RTN of the
source weights when no artifact exists, else the tensor is kept.
"""

from __future__ import annotations

import glob
import json
import logging
import os
import re

import numpy as np
import torch

from . import _native as nat
from .artifacts import ArtifactReader
from .grid import rtn_quantize_mxfp
from .packing import pack_q

log = logging.getLogger("mlx_gptq")

ROUTER_SKIP = r"(^|\.)(gate|router)$|shared_expert_gate"


def make_predicate(skip_regex, head_bits, embed_bits, group_size, mode="affine", path_bits=None):
    """mlx_lm.convert quantization predicate (pack.py:33-58)."""
    skip = re.compile(skip_regex) if skip_regex else None
    path_bits = path_bits or {}

    def predicate(path, module, *_):
        if skip and skip.search(path):
            return False
        if path in path_bits:
            return {"group_size": group_size, "bits": path_bits[path], "mode": mode}
        if path == "lm_head" or path.endswith(".lm_head"):
            return {"group_size": group_size, "bits": head_bits, "mode": mode} if head_bits else False
        if path.endswith("embed_tokens"):
            return {"group_size": group_size, "bits": embed_bits, "mode": mode} if embed_bits else False
        return True

    return predicate


def overrides_from_manifest(reader: ArtifactReader) -> dict[str, int]:
    """MLX module path -> bits for artifacts off the global width
    (pack.py:61-78); experts collapse onto their switch_mlp path."""
    global_bits = reader.manifest["bits"]
    out: dict[str, int] = {}
    for name, info in reader.tensors.items():
        if info["bits"] == global_bits:
            continue
        path = re.sub(r"\.experts\.\d+\.", ".switch_mlp.", name)
        path = path[: -len(".weight")] if path.endswith(".weight") else path
        prev = out.get(path)
        if prev is not None and prev != info["bits"]:
            raise RuntimeError(f"{path}: conflicting expert bits {prev} vs {info['bits']}")
        out[path] = info["bits"]
    return out


def _expert_artifact(mlx_key: str, e: int) -> str:
    """Artifact name of expert e of a fused MLX expert tensor (pack.py:81-87)."""
    if ".switch_mlp." in mlx_key:
        return mlx_key.replace(".switch_mlp.", f".experts.{e}.")
    if ".experts.switch_glu." in mlx_key:
        return mlx_key.replace(".experts.switch_glu.", f".experts.{e}.")
    raise ValueError(f"unrecognized fused-expert MLX key: {mlx_key}")


def _stack_on_device(parts: list[torch.Tensor], dev) -> torch.Tensor:
    out = torch.empty((len(parts), *parts[0].shape), dtype=parts[0].dtype, device=dev)
    for i, p in enumerate(parts):
        out[i].copy_(p, non_blocking=True)
    return out


def _load_shard(path: str) -> tuple[dict[str, torch.Tensor], dict]:
    from safetensors import safe_open

    with safe_open(path, "pt") as f:
        meta = f.metadata() or {}
        return {k: f.get_tensor(k) for k in f.keys()}, meta


def inject(mlx_path: str, reader: ArtifactReader):
    """Replace every calibrated tensor of the converted MLX model at
    `mlx_path` (pack.py:90-227). Returns (injected keys, RTN-kept keys)."""
    shard_files = sorted(glob.glob(os.path.join(mlx_path, "model*.safetensors")))
    shard_files = [f for f in shard_files if not f.endswith(".index.json")]
    with open(os.path.join(mlx_path, "config.json")) as f:
        config = json.load(f)
    qcfg = config.get("quantization")
    if not qcfg:
        raise RuntimeError("converted model has no quantization config")

    def cfg_for(path):
        entry = qcfg.get(path)
        if isinstance(entry, dict):
            return (entry.get("group_size", qcfg["group_size"]), entry.get("bits", qcfg["bits"]),
                    entry.get("mode", qcfg.get("mode", "affine")))
        return qcfg["group_size"], qcfg["bits"], qcfg.get("mode", "affine")

    dev = nat.device_for()
    used: set[str] = set()
    injected, rtn_kept = [], []

    def checked(name, b_mode):
        q, s, b, info = reader.get(name)
        group_size, bits, mode = b_mode
        artifact_mode = info.get("mode", "affine")
        if info["bits"] != bits or info["group_size"] != group_size or artifact_mode != mode:
            raise RuntimeError(
                f"{name}: artifact is {artifact_mode}/{info['bits']}b/g{info['group_size']} but "
                f"model config expects {mode}/{bits}b/g{group_size}; re-run convert with matching "
                "settings or fix overrides"
            )
        used.add(name)
        return q, s, b

    for shard in shard_files:
        weights, meta = _load_shard(shard)
        changed = False
        for key in list(weights.keys()):
            if not key.endswith(".weight") or f"{key[:-7]}.scales" not in weights:
                continue
            base = key[:-7]
            wq_old, s_old = weights[key], weights[f"{base}.scales"]
            group_size, bits, mode = cfg_for(base)
            if wq_old.dim() == 3 and (".switch_mlp." in key or ".experts.switch_glu." in key):
                E = wq_old.shape[0]
                arts = [_expert_artifact(key, e) for e in range(E)]
                missing = [a for a in arts if not reader.has(a)]
                if missing:
                    if len(missing) < E:
                        raise RuntimeError(f"{key}: only some experts have artifacts (e.g. {missing[0]})")
                    rtn_kept.append(key)
                    continue
                got = [checked(a, (group_size, bits, mode)) for a in arts]
                q_all = _stack_on_device([g[0] for g in got], dev)
                s_all = torch.stack([g[1] for g in got])
                bs = [g[2].float() for g in got if g[2] is not None]
                b_all = torch.stack(bs) if bs else None
            elif wq_old.dim() == 2 and reader.has(key):
                q_all, s_all, b = checked(key, (group_size, bits, mode))
                b_all = None if b is None else b.float()
            else:
                rtn_kept.append(key)
                continue
            words = pack_q(q_all.to(dev), bits).cpu()
            if tuple(words.shape) != tuple(wq_old.shape):
                raise RuntimeError(f"{key}: packed shape {tuple(words.shape)} != converted shape "
                                   f"{tuple(wq_old.shape)}")
            if tuple(s_all.shape) != tuple(s_old.shape):
                raise RuntimeError(f"{base}.scales: artifact shape {tuple(s_all.shape)} != "
                                   f"{tuple(s_old.shape)}")
            weights[key] = words.view(wq_old.dtype) if words.dtype != wq_old.dtype else words
            weights[f"{base}.scales"] = s_all.to(s_old.dtype)
            if mode == "affine":
                if b_all is None or f"{base}.biases" not in weights:
                    raise RuntimeError(f"{base}: affine artifact is missing biases")
                weights[f"{base}.biases"] = b_all.to(s_old.dtype)
            elif b_all is not None:
                raise RuntimeError(f"{base}: {mode} artifact unexpectedly has biases")
            injected.append(key)
            changed = True
        if changed:
            from safetensors.torch import save_file

            tmp = shard.replace(".safetensors", ".inject-tmp.safetensors")
            save_file({k: v.contiguous() for k, v in weights.items()}, tmp,
                      metadata={**meta, "format": "mlx"})
            os.replace(tmp, shard)
        del weights
        log.info("shard %s done", os.path.basename(shard))

    unused = [a for a in reader.tensors if a not in used]
    log.info("injected %d tensors; %d stayed RTN", len(injected), len(rtn_kept))
    if unused:
        raise RuntimeError(f"{len(unused)} artifacts were never consumed (naming mismatch?), "
                           f"e.g. {unused[:5]}")
    if not injected:
        raise RuntimeError("nothing was injected — check artifact naming vs model")
    return injected, rtn_kept


class ShardEmitter:
    """The streaming packer's per-tensor rule (stream_pack.py:139-221) for
    MXFP artifacts: stacked experts, one artifact, RTN, or kept."""

    def __init__(self, reader: ArtifactReader, mode: str, bits: int, group_size: int,
                 scale_dtype=np.uint8, storage_dtype=np.float16, exclude: str | None = None):
        self.reader = reader
        self.mode, self.bits, self.group_size = mode, bits, group_size
        self.scale_dtype, self.storage_dtype = scale_dtype, storage_dtype
        self.exclude = re.compile(exclude) if exclude else None
        self.used_artifacts: set[str] = set()
        self.stats = {"injected": 0, "rtn": 0, "kept": 0}

    def _quantizable(self, key: str, arr) -> bool:
        """stream_pack.py:139-153."""
        if not key.endswith(".weight") or arr.ndim not in (2, 3) or arr.shape[-1] % self.group_size:
            return False
        module_key = key.removesuffix(".weight")
        if module_key == "lm_head" or module_key.endswith(".lm_head"):
            return False
        if module_key.endswith("embed_tokens"):
            return False
        if self.exclude and self.exclude.search(module_key):
            return False
        return "ngram_embedding.shards." not in key

    def _get(self, name: str):
        q, s, b, info = self.reader.get(name)
        if info.get("bits") != self.bits or info.get("group_size") != self.group_size:
            raise RuntimeError(f"{name}: artifact {info['bits']}b/g{info['group_size']} != config "
                               f"{self.bits}b/g{self.group_size}")
        self.used_artifacts.add(name)
        return q, s, b

    def emit(self, mlx_key: str, arr) -> dict[str, np.ndarray]:
        """Output tensors for one source tensor `arr` (numpy or torch)."""
        base = mlx_key[: -len(".weight")]
        dev = nat.device_for()
        if arr.ndim == 3 and ".switch_mlp." in mlx_key:
            E = arr.shape[0]
            arts = [mlx_key.replace(".switch_mlp.", f".experts.{e}.") for e in range(E)]
            if all(self.reader.has(a) for a in arts):
                got = [self._get(a) for a in arts]
                words = pack_q(_stack_on_device([g[0] for g in got], dev), self.bits)
                scales = np.stack([g[1].numpy() for g in got])
                self.stats["injected"] += E
                return {f"{base}.weight": words.cpu().numpy().view(np.uint32),
                        f"{base}.scales": scales.astype(self.scale_dtype)}
        if self.reader.has(mlx_key) and self._quantizable(mlx_key, arr):
            q, s, b = self._get(mlx_key)
            out = {f"{base}.weight": pack_q(q.numpy(), self.bits),
                   f"{base}.scales": np.asarray(s.numpy()).astype(self.scale_dtype)}
            if b is not None:
                out[f"{base}.biases"] = np.asarray(b.float().numpy()).astype(self.storage_dtype)
            self.stats["injected"] += 1
            return out
        if self._quantizable(mlx_key, arr):
            w = torch.as_tensor(arr).to(dev, torch.float32)
            q, s, _b, _dq = rtn_quantize_mxfp(w.unsqueeze(0), self.mode)
            self.stats["rtn"] += 1
            return {f"{base}.weight": pack_q(q[0], self.bits).cpu().numpy().view(np.uint32),
                    f"{base}.scales": s[0].cpu().numpy().astype(self.scale_dtype)}
        self.stats["kept"] += 1
        return {mlx_key: arr}
