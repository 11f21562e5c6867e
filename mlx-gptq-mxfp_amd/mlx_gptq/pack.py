"""Stage-B shard emission on the Linux side: calibrated artifacts written
into MLX-layout shards, with code packing and the RTN fallback on the HIP
device. Behaviour follows the reference's ``pack.py`` (``make_predicate``,
``overrides_from_manifest``, ``inject``: pack.py:33-227) and the per-tensor
rule of ``stream_pack.py``'s ``StreamingPacker.emit`` (stream_pack.py:139-221).

Design. Every quantized tensor of a converted model is first resolved into
a ``_Target`` (the artifacts that feed it and the format the model's
``config.json`` expects for it); the artifacts are then fetched, checked
against that format, stacked on the device and packed in one ``mgq_pack_q``
launch per target; finally the words, scales and biases are spliced into the
shard after the shape checks. Shards are read and written with safetensors
(``"format": "mlx"`` metadata, as ``mlx.save_safetensors`` writes them), each
rewritten under a temporary name and renamed, so no MLX runtime is needed.

What stays the reference's: the file layout, the tensor names
(``{base}.weight`` / ``.scales`` / ``.biases``; per-expert artifact names
``...experts.{e}...``), the predicate's outcomes, and the error messages.
"""

from __future__ import annotations

import argparse
import glob
import json
import logging
import os
import re
from dataclasses import dataclass

import numpy as np
import torch

from . import _native as nat
from .artifacts import ArtifactReader
from .grid import rtn_quantize_mxfp
from .packing import pack_q

log = logging.getLogger("mlx_gptq")

# default --router-skip of the reference's Stage-B CLI: routers and shared
# expert gates stay unquantized
ROUTER_SKIP = r"(^|\.)(gate|router)$|shared_expert_gate"

# fused expert tensors of an MLX model and the per-expert artifact spelling
_FUSED_MARKERS = (".switch_mlp.", ".experts.switch_glu.")


# --------------------------------------------------------------------------
# convert-time policy
# --------------------------------------------------------------------------


class QuantPredicate:
    """``quant_predicate`` for ``mlx_lm.convert`` (pack.py:33-58).

    Outcome per module path: ``False`` (leave unquantized), ``True`` (the
    global settings) or ``{"group_size", "bits", "mode"}`` (own bits). The
    first matching rule wins: the skip regex; a per-path override; the LM
    head (quantized only with ``head_bits``); the token embedding (only with
    ``embed_bits``)."""

    def __init__(self, skip_regex, head_bits, embed_bits, group_size, mode="affine",
                 path_bits=None):
        self.skip = re.compile(skip_regex) if skip_regex else None
        self.group_size, self.mode = group_size, mode
        overrides = dict(path_bits or {})
        self.rules = (
            (lambda p: p in overrides, lambda p: overrides[p]),
            (lambda p: p == "lm_head" or p.endswith(".lm_head"), lambda p: head_bits),
            (lambda p: p.endswith("embed_tokens"), lambda p: embed_bits),
        )

    def __call__(self, path, module, *_):
        if self.skip is not None and self.skip.search(path):
            return False
        for matches, bits_of in self.rules:
            if matches(path):
                bits = bits_of(path)
                if not bits:
                    return False
                return {"group_size": self.group_size, "bits": bits, "mode": self.mode}
        return True


def make_predicate(skip_regex, head_bits, embed_bits, group_size, mode="affine", path_bits=None):
    """The convert predicate (pack.py:33-58); see ``QuantPredicate``."""
    return QuantPredicate(skip_regex, head_bits, embed_bits, group_size, mode, path_bits)


def _module_path(artifact_name: str) -> str:
    """MLX module path of an artifact: experts fold onto ``switch_mlp``."""
    path = re.sub(r"\.experts\.\d+\.", ".switch_mlp.", artifact_name)
    return path.removesuffix(".weight")


def overrides_from_manifest(reader: ArtifactReader) -> dict[str, int]:
    """MLX module path -> bits of every artifact off the manifest's global
    bits (pack.py:61-78); all experts of one fused path must agree."""
    default = reader.manifest["bits"]
    chosen: dict[str, int] = {}
    for name, info in reader.tensors.items():
        bits = info["bits"]
        if bits == default:
            continue
        path = _module_path(name)
        first = chosen.setdefault(path, bits)
        if first != bits:
            raise RuntimeError(f"{path}: conflicting expert bits {first} vs {bits}")
    return chosen


# --------------------------------------------------------------------------
# injection into a converted model
# --------------------------------------------------------------------------


class _QuantConfig:
    """config.json's "quantization" block: global settings plus per-module
    dict entries that override them."""

    def __init__(self, config: dict):
        q = config.get("quantization")
        if not q:
            raise RuntimeError("converted model has no quantization config")
        self.default = (q["group_size"], q["bits"], q.get("mode", "affine"))
        self.per_module = {k: v for k, v in q.items() if isinstance(v, dict)}

    def format_of(self, base: str) -> tuple[int, int, str]:
        entry = self.per_module.get(base)
        if entry is None:
            return self.default
        g, b, m = self.default
        return entry.get("group_size", g), entry.get("bits", b), entry.get("mode", m)


@dataclass
class _Target:
    key: str                     # "{base}.weight" in the shard
    artifacts: list[str]         # one per expert for a fused tensor, else one
    fmt: tuple[int, int, str]    # (group_size, bits, mode) the model expects
    fused: bool

    @property
    def base(self) -> str:
        return self.key[: -len(".weight")]


def _expert_names(key: str, experts: int) -> list[str] | None:
    marker = next((m for m in _FUSED_MARKERS if m in key), None)
    if marker is None:
        return None
    return [key.replace(marker, f".experts.{e}.") for e in range(experts)]


def _resolve(key: str, shape: tuple, cfg: _QuantConfig, reader: ArtifactReader):
    """The _Target feeding `key`, or None when it keeps its RTN codes."""
    fmt = cfg.format_of(key[: -len(".weight")])
    names = _expert_names(key, shape[0]) if len(shape) == 3 else None
    if names is not None:
        present = [reader.has(a) for a in names]
        if all(present):
            return _Target(key, names, fmt, True)
        if any(present):
            missing = names[present.index(False)]
            raise RuntimeError(f"{key}: only some experts have artifacts (e.g. {missing})")
        return None
    if len(shape) == 2 and reader.has(key):
        return _Target(key, [key], fmt, False)
    return None


def _format_error(t: _Target, name: str, info: dict) -> str:
    g, b, m = t.fmt
    got = f"{info.get('mode', 'affine')}/{info['bits']}b/g{info['group_size']}"
    if t.fused:
        return (f"{name}: artifact is {got} but model config expects {m}/{b}b/g{g}; "
                "re-run convert with matching settings or fix overrides")
    return f"{name}: artifact {got} vs config {m}/{b}b/g{g}"


def _fetch(t: _Target, reader: ArtifactReader, dev):
    """Codes (stacked on the device for a fused target), scales and biases of
    a target, each artifact checked against the model's format."""
    g, b, m = t.fmt
    codes, scales, biases = [], [], []
    for name in t.artifacts:
        q, s, bias, info = reader.get(name)
        if (info["bits"], info["group_size"], info.get("mode", "affine")) != (b, g, m):
            raise RuntimeError(_format_error(t, name, info))
        codes.append(q)
        scales.append(s)
        if bias is not None:
            biases.append(bias.float())
    if not t.fused:
        return codes[0].to(dev), scales[0], biases[0] if biases else None
    q_all = torch.empty((len(codes), *codes[0].shape), dtype=torch.uint8, device=dev)
    for i, q in enumerate(codes):
        q_all[i].copy_(q, non_blocking=True)
    return q_all, torch.stack(scales), torch.stack(biases) if biases else None


def _splice(weights: dict, t: _Target, words: torch.Tensor, scales, biases) -> None:
    """Put a target's packed words, scales and biases into the shard dict."""
    old_w, old_s = weights[t.key], weights[f"{t.base}.scales"]
    if tuple(words.shape) != tuple(old_w.shape):
        raise RuntimeError(f"{t.key}: packed shape {tuple(words.shape)} != converted shape "
                           f"{tuple(old_w.shape)}")
    if tuple(scales.shape) != tuple(old_s.shape):
        raise RuntimeError(f"{t.base}.scales: artifact shape {tuple(scales.shape)} != "
                           f"{tuple(old_s.shape)}")
    mode = t.fmt[2]
    if mode == "affine" and (biases is None or f"{t.base}.biases" not in weights):
        raise RuntimeError(f"{t.base}: affine artifact is missing biases")
    if mode != "affine" and biases is not None:
        raise RuntimeError(f"{t.base}: {mode} artifact unexpectedly has biases")
    weights[t.key] = words if words.dtype == old_w.dtype else words.view(old_w.dtype)
    weights[f"{t.base}.scales"] = scales.to(old_s.dtype)
    if biases is not None:
        weights[f"{t.base}.biases"] = biases.to(old_s.dtype)


def _shard_files(mlx_path: str) -> list[str]:
    files = sorted(glob.glob(os.path.join(mlx_path, "model*.safetensors")))
    return [f for f in files if not f.endswith(".index.json")]


def _rewrite_shard(path: str, weights: dict, metadata: dict) -> None:
    from safetensors.torch import save_file

    tmp = path.replace(".safetensors", ".inject-tmp.safetensors")
    save_file({k: v.contiguous() for k, v in weights.items()}, tmp,
              metadata={**metadata, "format": "mlx"})
    os.replace(tmp, path)


def inject(mlx_path: str, reader: ArtifactReader):
    """Replace every calibrated tensor of the converted MLX model at
    `mlx_path` with its artifact (pack.py:90-227). Returns (injected keys,
    keys that keep their RTN codes). Raises if an artifact is never used or
    nothing was injected."""
    from safetensors import safe_open

    with open(os.path.join(mlx_path, "config.json")) as f:
        cfg = _QuantConfig(json.load(f))
    dev = nat.device_for()
    consumed: set[str] = set()
    injected, kept = [], []
    for shard in _shard_files(mlx_path):
        with safe_open(shard, "pt") as f:
            metadata = f.metadata() or {}
            weights = {k: f.get_tensor(k) for k in f.keys()}
        targets = []
        for key, w in weights.items():
            if not key.endswith(".weight") or f"{key[:-7]}.scales" not in weights:
                continue
            t = _resolve(key, tuple(w.shape), cfg, reader)
            (kept.append(key) if t is None else targets.append(t))
        for t in targets:
            q, scales, biases = _fetch(t, reader, dev)
            words = pack_q(q, t.fmt[1]).cpu()
            _splice(weights, t, words, scales, biases)
            consumed.update(t.artifacts)
            injected.append(t.key)
        if targets:
            _rewrite_shard(shard, weights, metadata)
        log.info("shard %s done", os.path.basename(shard))
    log.info("injected %d tensors; %d stayed RTN", len(injected), len(kept))
    unused = [a for a in reader.tensors if a not in consumed]
    if unused:
        raise RuntimeError(f"{len(unused)} artifacts were never consumed (naming mismatch?), "
                           f"e.g. {unused[:5]}")
    if not injected:
        raise RuntimeError("nothing was injected — check artifact naming vs model")
    return injected, kept


# --------------------------------------------------------------------------
# streaming emission (one source tensor at a time)
# --------------------------------------------------------------------------


class ShardEmitter:
    """Per-tensor emission rule of the reference's streaming packer
    (stream_pack.py:139-221) for MXFP checkpoints. ``emit(key, arr)`` returns
    the MLX tensors that replace source tensor `arr`: the stacked experts'
    artifacts, the tensor's own artifact, MXFP RTN of the source weights
    when a quantizable tensor has none, or the tensor unchanged."""

    def __init__(self, reader: ArtifactReader, mode: str, bits: int, group_size: int,
                 scale_dtype=np.uint8, storage_dtype=np.float16, exclude: str | None = None):
        self.reader = reader
        self.mode, self.bits, self.group_size = mode, bits, group_size
        self.scale_dtype, self.storage_dtype = scale_dtype, storage_dtype
        self.exclude = re.compile(exclude) if exclude else None
        self.used_artifacts: set[str] = set()
        self.stats = {"injected": 0, "rtn": 0, "kept": 0}

    def quantizable(self, key: str, arr) -> bool:
        """A 2D/3D ``.weight`` whose rows split into groups, other than the
        LM head, the token embedding, excluded modules and n-gram shards."""
        if not key.endswith(".weight") or arr.ndim not in (2, 3) or arr.shape[-1] % self.group_size:
            return False
        module = key[: -len(".weight")]
        excluded = (
            module == "lm_head" or module.endswith(".lm_head"),
            module.endswith("embed_tokens"),
            self.exclude is not None and bool(self.exclude.search(module)),
            "ngram_embedding.shards." in key,
        )
        return not any(excluded)

    def _artifact(self, name: str):
        q, s, b, info = self.reader.get(name)
        if info.get("bits") != self.bits or info.get("group_size") != self.group_size:
            raise RuntimeError(f"{name}: artifact {info['bits']}b/g{info['group_size']} != config "
                               f"{self.bits}b/g{self.group_size}")
        self.used_artifacts.add(name)
        return q, s, b

    def _route(self, key: str, arr):
        if arr.ndim == 3 and ".switch_mlp." in key:
            names = [key.replace(".switch_mlp.", f".experts.{e}.") for e in range(arr.shape[0])]
            if all(self.reader.has(a) for a in names):
                return "experts", names
        if not self.quantizable(key, arr):
            return "keep", None
        return ("artifact", [key]) if self.reader.has(key) else ("rtn", None)

    def emit(self, mlx_key: str, arr) -> dict[str, np.ndarray]:
        route, names = self._route(mlx_key, arr)
        base = mlx_key[: -len(".weight")] if mlx_key.endswith(".weight") else mlx_key
        if route == "keep":
            self.stats["kept"] += 1
            return {mlx_key: arr}
        dev = nat.device_for()
        biases = None
        if route == "rtn":
            w = torch.as_tensor(arr).to(dev, torch.float32).unsqueeze(0)
            q, scales, _, _ = rtn_quantize_mxfp(w, self.mode)
            q, scales = q[0], scales[0].cpu()
            self.stats["rtn"] += 1
        else:
            got = [self._artifact(a) for a in names]
            if route == "experts":
                q = torch.stack([g[0] for g in got]).to(dev)
                scales = torch.stack([g[1] for g in got])
            else:
                (q, scales, biases), = got
                q = q.to(dev)
            self.stats["injected"] += len(names)
        out = {f"{base}.weight": pack_q(q, self.bits).cpu().numpy().view(np.uint32),
               f"{base}.scales": np.asarray(scales.numpy()).astype(self.scale_dtype)}
        if biases is not None:
            out[f"{base}.biases"] = np.asarray(biases.float().numpy()).astype(self.storage_dtype)
        return out


# --------------------------------------------------------------------------
# CLI (the reference's Stage-B command line; the convert step needs mlx_lm)
# --------------------------------------------------------------------------


def main(argv=None):
    """``python -m mlx_gptq.pack``: RTN-convert with mlx_lm (unless
    --skip-convert), then inject the artifacts."""
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--hf-path", required=True, help="original HF model (id or dir)")
    ap.add_argument("--calib", required=True, help="Stage A artifact dir")
    ap.add_argument("--mlx-path", required=True, help="output MLX model dir")
    ap.add_argument("--skip-convert", action="store_true",
                    help="mlx-path already holds a converted RTN model; only inject")
    ap.add_argument("--router-skip", default=ROUTER_SKIP,
                    help="regex of module paths to leave unquantized during convert")
    ap.add_argument("--head-bits", type=int, default=None,
                    help="RTN bits for lm_head (default: global bits)")
    ap.add_argument("--embed-bits", type=int, default=None)
    ap.add_argument("--trust-remote-code", action="store_true")
    ap.add_argument("--verify", action="store_true", help="load and generate afterwards")
    args = ap.parse_args(argv)
    logging.basicConfig(level=logging.INFO, format="%(asctime)s %(levelname)s %(message)s",
                        datefmt="%H:%M:%S")
    reader = ArtifactReader(args.calib)
    m = reader.manifest
    mode = m.get("mode", "affine")
    if not args.skip_convert:
        from mlx_lm.convert import convert  # Apple-side dependency

        convert(args.hf_path, mlx_path=args.mlx_path, quantize=True, q_group_size=m["group_size"],
                q_bits=m["bits"], q_mode=mode, dtype=m["storage_dtype"],
                quant_predicate=make_predicate(args.router_skip, args.head_bits, args.embed_bits,
                                               m["group_size"], mode=mode,
                                               path_bits=overrides_from_manifest(reader)),
                trust_remote_code=args.trust_remote_code)
    inject(args.mlx_path, reader)
    if args.verify:
        from mlx_lm import generate, load

        model, tokenizer = load(args.mlx_path)
        log.info("verify generate: %s", generate(model, tokenizer,
                                                 prompt="The capital of France is", max_tokens=40))


if __name__ == "__main__":
    main()
