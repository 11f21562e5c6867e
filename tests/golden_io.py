"""Loader for the committed golden vectors (safetensors + JSON, data only)."""

from __future__ import annotations

import json
import os

import torch
from safetensors.torch import load_file

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load():
    tensors = load_file(os.path.join(HERE, "solver_golden.safetensors"))
    with open(os.path.join(HERE, "solver_golden.json")) as f:
        meta = json.load(f)
    return tensors, meta


def case_kwargs(kw: dict) -> dict:
    out = dict(kw)
    if "storage_dtype" in out:
        out["storage_dtype"] = getattr(torch, out["storage_dtype"].split(".")[-1])
    return out
