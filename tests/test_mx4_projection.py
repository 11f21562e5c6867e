"""Exhaustive CPU check of the solver's MXFP4 arithmetic over all 2^32 fp32
inputs, against the threshold-chain encoder e2m1_code / e2m1_value (the
grid.py:82-105 restatement in csrc/mgq_common.h): the compare-free exact
encoder mx4_encode (code and dq) and the quantization error mx4_err used to
score safe-scale-search candidates. Compiles the header for the host with
hipcc."""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(HERE), "mlx-gptq-mxfp_amd", "csrc")


def _hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    return None


@pytest.mark.skipif(_hipcc() is None, reason="hipcc not available")
def test_mx4_fast_projection_exhaustive(tmp_path):
    exe = tmp_path / "check_mx4"
    subprocess.run([_hipcc(), "-O2", "-std=c++17", "-I", CSRC,
                    os.path.join(HERE, "native", "check_mx4_projection.hip"), "-o", str(exe)],
                   check=True, capture_output=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "mismatches=0" in res.stdout
