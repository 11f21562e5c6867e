"""Build libmlxgptq_hip.so (gfx950) in-tree from csrc/*.hip with hipcc.

Usage: python build.py [--jobs N] [--verbose]

Objects go to ``_build/`` beside this file; the shared library lands in
``mlx_gptq/libmlxgptq_hip.so`` where ``mlx_gptq._native`` loads it. Every call
recompiles (the driver's "does it build" check relies on that).
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
OUT = HERE / "mlx_gptq" / "libmlxgptq_hip.so"
ARCH = "gfx950"
# Test-only GPU library: the exhaustive check of the hardware MX conversion
# forms (csrc/mx_hw.h) that tests/test_gpu_mx_hw.py runs.
HWCHECK_SRC = HERE.parent / "tests" / "native" / "check_mx_hw.hip"
HWCHECK_OUT = HERE.parent / "tests" / "native" / "libmgq_hwcheck.so"

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # torch evaluates `a*b + c` as two roundings; keep every encode path IEEE.
    "-ffp-contract=off",
    # Packed fp32 VALU ops have given silent wrong results on these boxes.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wno-unused-result",
]


# Per-source extra flags. The MXFP solver's candidate objective keeps its
# small MFMA accumulators in ordinary VGPRs (they feed VALU code right away);
# the Hessian kernel keeps the default, which puts its 256 accumulators in
# AGPRs.
EXTRA_FLAGS = {"gptq_mxfp.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm required to build libmlxgptq_hip.so)")


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-I", str(CSRC), "-c", str(src),
           "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(8, len(sources), os.cpu_count() or 1)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources))
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, OUT)
    if HWCHECK_SRC.exists():
        _build_hwcheck(verbose)
    return OUT


def _build_hwcheck(verbose: bool) -> None:
    tmp = HWCHECK_OUT.with_suffix(".so.tmp")
    cmd = [hipcc(), *COMMON_FLAGS, "-shared", "-I", str(CSRC), str(HWCHECK_SRC), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {HWCHECK_SRC.name}:\n{res.stderr}")
    os.replace(tmp, HWCHECK_OUT)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--verbose", action="store_true")
    args = ap.parse_args(argv)
    out = build(args.jobs, args.verbose)
    print(out)
    return 0


if __name__ == "__main__":
    sys.exit(main())
