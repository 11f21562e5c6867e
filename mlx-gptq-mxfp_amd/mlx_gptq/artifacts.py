"""Calibration artifact store (artifacts.py API) on MI355X.

Directory layout, the same as the reference's (artifacts.py:1-15) so that
either side's reader takes either side's output:

    calib_dir/
      manifest.json            header + "tensors" (per-tensor metadata) + "layers_done"
      layer_0000.safetensors   {name}.q / {name}.scales / optional {name}.biases
      ...

4-bit codes are stored nibble-packed, two per byte, low nibble first
(``"q_packed": "nibble"``), other widths raw. ``ArtifactWriter.write_layer``
takes the solver's device tensors as they are: the 4-bit codes are packed on
the device (csrc/pack.hip), every tensor of the layer is copied into pinned
host memory with one synchronisation, and the layer file is written under a
temporary name and renamed. The manifest is rewritten atomically after each
layer, as the reference does.
"""

from __future__ import annotations

import json
import os
import tempfile

import torch

from . import _native as nat

_STR_TO_DTYPE = {"bfloat16": torch.bfloat16, "float16": torch.float16}
_RESUME_KEYS = ("mode", "bits", "group_size", "storage_dtype")


def pack_nibbles(q: torch.Tensor) -> torch.Tensor:
    """uint8 [..., C] -> uint8 [..., C/2] with byte = q[2k] | q[2k+1] << 4 (artifacts.py:30-32)."""
    assert q.dtype == torch.uint8 and q.shape[-1] % 2 == 0
    dev = nat.device_for(q)
    x = nat.on_device(q, dev)
    *lead, C = q.shape
    rows = nat.numel_groups(tuple(lead))
    out = torch.empty((*lead, C // 2), dtype=torch.uint8, device=dev)
    if rows and C:
        nat.call("mgq_pack_nibbles", x.data_ptr(), rows, C, out.data_ptr(), nat.stream_of(dev))
    return out.to(q.device)


def unpack_nibbles(p: torch.Tensor) -> torch.Tensor:
    """uint8 [..., P] -> uint8 [..., 2P], low nibble first (artifacts.py:35-39)."""
    dev = nat.device_for(p)
    x = nat.on_device(p.to(torch.uint8), dev)
    *lead, P = p.shape
    rows = nat.numel_groups(tuple(lead))
    out = torch.empty((*lead, 2 * P), dtype=torch.uint8, device=dev)
    if rows and P:
        nat.call("mgq_unpack_nibbles", x.data_ptr(), rows, P, out.data_ptr(), nat.stream_of(dev))
    return out.to(p.device)


def _to_host(tensors: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """Contiguous CPU copies; device tensors go through pinned buffers with
    one synchronisation for the whole set."""
    out, pending, seen = {}, False, set()
    for k, t in tensors.items():
        t = t.detach()
        if t.is_cuda:
            h = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
            h.copy_(t.contiguous(), non_blocking=True)
            out[k] = h
            pending = True
        else:
            t = t.contiguous()
            # safetensors refuses two names over one buffer
            if t.numel() and t.untyped_storage().data_ptr() in seen:
                t = t.clone()
            seen.add(t.untyped_storage().data_ptr())
            out[k] = t
    if pending:
        torch.cuda.synchronize()
    return out


class ArtifactWriter:
    """Stage-A artifact store (artifacts.py:42-102): same manifest keys,
    resume check and file names."""

    def __init__(self, out_dir: str, header: dict):
        self.dir = out_dir
        os.makedirs(out_dir, exist_ok=True)
        self.manifest_path = os.path.join(out_dir, "manifest.json")
        if os.path.exists(self.manifest_path):
            with open(self.manifest_path) as f:
                self.manifest = json.load(f)
            for k, v in header.items():
                if k in _RESUME_KEYS and self.manifest.get(k) != v:
                    raise RuntimeError(
                        f"resume mismatch: manifest has {k}={self.manifest.get(k)}, run has {v}"
                    )
        else:
            self.manifest = dict(header)
            self.manifest["tensors"] = {}
            self.manifest["layers_done"] = []

    def layer_done(self, layer_idx: int) -> bool:
        return layer_idx in self.manifest["layers_done"]

    def layer_file(self, layer_idx: int) -> str:
        return os.path.join(self.dir, f"layer_{layer_idx:04d}.safetensors")

    def write_layer(self, layer_idx: int, tensors: dict, meta: dict):
        """tensors: name -> (q uint8 [out, in], scales, optional biases), on a
        HIP device or the host; meta: name -> metadata with at least "bits"
        (updated in place with "q_packed", "has_biases" and "file")."""
        from safetensors.torch import save_file

        fname = f"layer_{layer_idx:04d}.safetensors"
        flat = {}
        for name, (q, s, b) in tensors.items():
            if meta[name]["bits"] == 4:
                q = pack_nibbles(q)
                meta[name]["q_packed"] = "nibble"
            else:
                meta[name]["q_packed"] = "raw"
            flat[f"{name}.q"] = q
            flat[f"{name}.scales"] = s
            meta[name]["has_biases"] = b is not None
            if b is not None:
                flat[f"{name}.biases"] = b
            meta[name]["file"] = fname
        flat = _to_host(flat)
        fd, tmp = tempfile.mkstemp(dir=self.dir, suffix=".safetensors.tmp")
        os.close(fd)
        try:
            save_file(flat, tmp)
            os.replace(tmp, self.layer_file(layer_idx))
        except BaseException:
            if os.path.exists(tmp):
                os.unlink(tmp)
            raise
        self.manifest["tensors"].update(meta)
        self.manifest["layers_done"].append(layer_idx)
        self._flush()

    def _flush(self):
        fd, tmp = tempfile.mkstemp(dir=self.dir, suffix=".json.tmp")
        with os.fdopen(fd, "w") as f:
            json.dump(self.manifest, f)
        os.replace(tmp, self.manifest_path)


class ArtifactReader:
    """Stage-B reader (artifacts.py:105-139). ``get`` returns host tensors,
    the 4-bit codes unpacked (on the HIP device)."""

    def __init__(self, calib_dir: str):
        self.dir = calib_dir
        with open(os.path.join(calib_dir, "manifest.json")) as f:
            self.manifest = json.load(f)
        self.tensors = self.manifest["tensors"]
        self._cache_file = None
        self._cache = None

    @property
    def storage_dtype(self) -> torch.dtype:
        return _STR_TO_DTYPE[self.manifest["storage_dtype"]]

    def has(self, name: str) -> bool:
        return name in self.tensors

    def _load(self, fname: str) -> dict:
        from safetensors.torch import load_file

        if self._cache_file != fname:
            self._cache = load_file(os.path.join(self.dir, fname))
            self._cache_file = fname
        return self._cache

    def get(self, name: str):
        """(q uint8 [out, in], scales, optional biases, info)."""
        info = self.tensors[name]
        blob = self._load(info["file"])
        q = blob[f"{name}.q"]
        if info["q_packed"] == "nibble":
            q = unpack_nibbles(q)
        return q, blob[f"{name}.scales"], blob.get(f"{name}.biases"), info
