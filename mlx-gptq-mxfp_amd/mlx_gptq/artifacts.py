"""Calibration artifact store (the reference's artifacts.py API) on MI355X.

On-disk format, shared with the reference (artifacts.py:1-15) so that either
side reads the other's output:

    calib_dir/
      manifest.json            run header + "tensors" {name: info} + "layers_done" [int]
      layer_0000.safetensors   {name}.q / {name}.scales / optional {name}.biases
      ...

``info`` carries the solver's metadata plus three storage fields:
``"q_packed"`` ("nibble": 4-bit codes two per byte, low nibble first;
"raw": one code per byte), ``"has_biases"`` and ``"file"``.

Design:

* ``_Manifest`` owns the JSON document: resume validation against the run
  header, and atomic replacement (temporary file + rename) on every save.
* Codes are encoded by a per-bit-width codec (``_CODECS``); 4-bit packing
  runs on the HIP device (``mgq_pack_nibbles``), so ``write_layer`` takes the
  solver's device tensors as they are. The layer's tensors are staged into
  pinned host buffers and synchronised once, and the layer file is written
  under a temporary name and renamed.
* ``ArtifactReader`` opens layer files lazily with ``safe_open`` and reads
  only the tensors asked for (a few handles kept open, least recently used
  closed first) instead of loading whole layer files.
"""

from __future__ import annotations

import json
import os
import tempfile
from collections import OrderedDict

import torch

from . import _native as nat

_STORAGE_DTYPES = {"bfloat16": torch.bfloat16, "float16": torch.float16}

# header fields a resumed run must agree on; the message is the reference's
_RESUME_FIELDS = ("mode", "bits", "group_size", "storage_dtype")


def _nibble_kernel(name: str, src: torch.Tensor, out_last: int) -> torch.Tensor:
    """Run one of the byte <-> nibble kernels over the last axis of `src`."""
    dev = nat.device_for(src)
    x = nat.on_device(src.to(torch.uint8), dev)
    *lead, n = src.shape
    rows = nat.numel_groups(tuple(lead))
    out = torch.empty((*lead, out_last), dtype=torch.uint8, device=dev)
    if rows and n:
        nat.call(name, x.data_ptr(), rows, n, out.data_ptr(), nat.stream_of(dev))
    return out.to(src.device)


def pack_nibbles(q: torch.Tensor) -> torch.Tensor:
    """uint8 [..., C] -> uint8 [..., C/2], byte k = q[2k] | q[2k+1] << 4
    (artifacts.py:30-32)."""
    assert q.dtype == torch.uint8 and q.shape[-1] % 2 == 0
    return _nibble_kernel("mgq_pack_nibbles", q, q.shape[-1] // 2)


def unpack_nibbles(p: torch.Tensor) -> torch.Tensor:
    """uint8 [..., P] -> uint8 [..., 2P], low nibble first (artifacts.py:35-39)."""
    return _nibble_kernel("mgq_unpack_nibbles", p, 2 * p.shape[-1])


# bits -> (q_packed tag, encode, decode); widths not listed are stored raw
_CODECS = {4: ("nibble", pack_nibbles, unpack_nibbles)}
_RAW = ("raw", lambda q: q, lambda q: q)
_DECODERS = {tag: dec for tag, _, dec in (*_CODECS.values(), _RAW)}


class _Manifest:
    """manifest.json of one artifact directory."""

    def __init__(self, directory: str, header: dict | None):
        self.path = os.path.join(directory, "manifest.json")
        self.dir = directory
        if os.path.exists(self.path):
            with open(self.path) as f:
                self.doc = json.load(f)
            for key in _RESUME_FIELDS:
                if header is not None and key in header and self.doc.get(key) != header[key]:
                    raise RuntimeError(
                        f"resume mismatch: manifest has {key}={self.doc.get(key)}, "
                        f"run has {header[key]}"
                    )
        elif header is None:
            raise FileNotFoundError(self.path)
        else:
            self.doc = {**header, "tensors": {}, "layers_done": []}

    def record_layer(self, layer_idx: int, infos: dict) -> None:
        self.doc["tensors"].update(infos)
        self.doc["layers_done"].append(layer_idx)
        self.save()

    def save(self) -> None:
        fd, tmp = tempfile.mkstemp(dir=self.dir, suffix=".json.tmp")
        with os.fdopen(fd, "w") as f:
            json.dump(self.doc, f)
        os.replace(tmp, self.path)


def _stage_to_host(tensors: dict[str, torch.Tensor]) -> dict[str, torch.Tensor]:
    """Contiguous host copies: device tensors through pinned buffers with one
    synchronisation for the whole set; host tensors that share storage are
    cloned (safetensors refuses aliases)."""
    staged, on_device, storages = {}, False, set()
    for key, t in tensors.items():
        t = t.detach()
        if t.is_cuda:
            host = torch.empty(t.shape, dtype=t.dtype, pin_memory=True)
            host.copy_(t.contiguous(), non_blocking=True)
            on_device = True
        else:
            host = t.contiguous()
            sid = host.untyped_storage().data_ptr()
            if host.numel() and sid in storages:
                host = host.clone()
            storages.add(host.untyped_storage().data_ptr())
        staged[key] = host
    if on_device:
        torch.cuda.synchronize()
    return staged


def _atomic_save(flat: dict[str, torch.Tensor], path: str) -> None:
    from safetensors.torch import save_file

    fd, tmp = tempfile.mkstemp(dir=os.path.dirname(path), suffix=".safetensors.tmp")
    os.close(fd)
    try:
        save_file(flat, tmp)
        os.replace(tmp, path)
    except BaseException:
        if os.path.exists(tmp):
            os.unlink(tmp)
        raise


class ArtifactWriter:
    """Stage-A side of the store (artifacts.py:42-102)."""

    def __init__(self, out_dir: str, header: dict):
        os.makedirs(out_dir, exist_ok=True)
        self.dir = out_dir
        self._m = _Manifest(out_dir, header)
        self.manifest_path = self._m.path

    @property
    def manifest(self) -> dict:
        return self._m.doc

    def layer_done(self, layer_idx: int) -> bool:
        return layer_idx in self._m.doc["layers_done"]

    def layer_file(self, layer_idx: int) -> str:
        return os.path.join(self.dir, f"layer_{layer_idx:04d}.safetensors")

    def write_layer(self, layer_idx: int, tensors: dict, meta: dict):
        """tensors: name -> (q uint8 [out, in], scales, biases or None), on a
        HIP device or the host; meta: name -> info with at least "bits",
        completed in place with the storage fields."""
        fname = os.path.basename(self.layer_file(layer_idx))
        flat = {}
        for name, (q, scales, biases) in tensors.items():
            info = meta[name]
            tag, encode, _ = _CODECS.get(info["bits"], _RAW)
            flat[f"{name}.q"] = encode(q)
            flat[f"{name}.scales"] = scales
            if biases is not None:
                flat[f"{name}.biases"] = biases
            info.update(q_packed=tag, has_biases=biases is not None, file=fname)
        _atomic_save(_stage_to_host(flat), self.layer_file(layer_idx))
        self._m.record_layer(layer_idx, meta)


class ArtifactReader:
    """Stage-B side of the store (artifacts.py:105-126). ``get`` returns host
    tensors; 4-bit codes are unpacked on the HIP device."""

    def __init__(self, calib_dir: str, open_files: int = 4):
        self.dir = calib_dir
        self.manifest = _Manifest(calib_dir, None).doc
        self.tensors = self.manifest["tensors"]
        self._handles: OrderedDict[str, object] = OrderedDict()
        self._open_files = max(1, int(open_files))

    @property
    def storage_dtype(self) -> torch.dtype:
        return _STORAGE_DTYPES[self.manifest["storage_dtype"]]

    def has(self, name: str) -> bool:
        return name in self.tensors

    def _file(self, fname: str):
        from safetensors import safe_open

        entry = self._handles.get(fname)
        if entry is None:
            h = safe_open(os.path.join(self.dir, fname), "pt")
            entry = (h, frozenset(h.keys()))
            self._handles[fname] = entry
            while len(self._handles) > self._open_files:
                self._handles.popitem(last=False)
        else:
            self._handles.move_to_end(fname)
        return entry

    def get(self, name: str):
        """(q uint8 [out, in], scales, biases or None, info)."""
        info = self.tensors[name]
        f, keys = self._file(info["file"])
        q = _DECODERS[info["q_packed"]](f.get_tensor(f"{name}.q"))
        biases = f.get_tensor(f"{name}.biases") if f"{name}.biases" in keys else None
        return q, f.get_tensor(f"{name}.scales"), biases, info
