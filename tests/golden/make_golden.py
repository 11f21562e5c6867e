"""Write golden input/output vectors for the solver by running the reference.

Run ONCE in the build container (where the reference checkout exists):

    python tests/golden/make_golden.py /root/reference

It imports the reference's own ``mlx_gptq`` package (solver modules only:
gptq.py, grid.py) and records, for small seeded inputs, the outputs of the
functions that no closed form pins bit for bit: ``solve_gptq`` in every mode
and algorithm (op-order-sensitive column recurrences and argmins),
``_prepare_hinv`` including damping escalation and its failure message, and
``choose_qparams`` (strict-< argmin over the shrink grid). The outputs are
saved as data (safetensors + JSON) next to this script; nothing of the
reference's source is stored.
"""

from __future__ import annotations

import json
import logging
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

OUT = Path(__file__).resolve().parent


def _setup(B, R, C, N, seed):
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(N, C, generator=g)
    X = base + 0.5 * torch.roll(base, 1, dims=1)
    scale = torch.exp(torch.randn(C, generator=g) * 0.5)
    X = X * scale
    W = torch.randn(B, R, C, generator=g) * 0.02
    H = (X.T @ X).unsqueeze(0).repeat(B, 1, 1)
    for b in range(1, B):
        H[b] *= 1.0 + 0.5 * b
    return W.contiguous(), H.contiguous()


CASES = [
    # name, B, R, C, N, seed, kwargs
    ("mxfp4_safe", 2, 16, 96, 512, 1, dict(bits=4, group_size=32, mode="mxfp4", mxfp_algorithm="safe-scale-search")),
    ("mxfp4_groupwise", 2, 16, 96, 512, 2, dict(bits=4, group_size=32, mode="mxfp4", mxfp_algorithm="groupwise")),
    ("mxfp8_groupwise", 2, 16, 96, 512, 3, dict(bits=8, group_size=32, mode="mxfp8", mxfp_algorithm="groupwise")),
    ("mxfp8_safe", 1, 16, 64, 512, 4, dict(bits=8, group_size=32, mode="mxfp8", mxfp_algorithm="safe-scale-search")),
    ("affine4_g64", 1, 16, 256, 1024, 5, dict(bits=4, group_size=64)),
    ("affine4_g32_f32", 2, 8, 128, 512, 6, dict(bits=4, group_size=32, storage_dtype=torch.float32)),
    ("affine2_g32", 1, 8, 192, 512, 7, dict(bits=2, group_size=32)),
    ("affine8_g128_minmax", 1, 8, 256, 512, 8, dict(bits=8, group_size=128, clip="minmax")),
]


def main(ref_root: str) -> int:
    sys.path.insert(0, ref_root)
    from mlx_gptq import gptq as rg  # the reference solver
    from mlx_gptq import grid as rgrid

    meta: dict = {"torch": torch.__version__, "cases": {}}
    tensors: dict[str, torch.Tensor] = {}

    for name, B, R, C, N, seed, kw in CASES:
        W, H = _setup(B, R, C, N, seed)
        if name.startswith("mxfp4_safe"):
            H[:, 5, :] = 0.0  # one dead column (zero row/col) in every item
            H[:, :, 5] = 0.0
        if name == "affine4_g64":
            H[0, 70, :] = 0.0
            H[0, :, 70] = 0.0
        W_in, H_in = W.clone(), H.clone()
        q, s, b, W_dq, rel = rg.solve_gptq(W, H, **kw)
        kw_json = {k: (str(v) if isinstance(v, torch.dtype) else v) for k, v in kw.items()}
        meta["cases"][name] = kw_json
        tensors[f"{name}.W"] = W_in
        tensors[f"{name}.H"] = H_in
        tensors[f"{name}.H_after"] = H.clone()
        tensors[f"{name}.q"] = q
        tensors[f"{name}.scales"] = s
        if b is not None:
            tensors[f"{name}.biases"] = b
        tensors[f"{name}.W_dq"] = W_dq
        tensors[f"{name}.rel"] = rel

    # _prepare_hinv: escalation that recovers, and one that raises.
    g = torch.Generator().manual_seed(11)
    A = torch.randn(4, 32, 32, generator=g)
    Hs = A @ A.transpose(1, 2) + 0.1 * torch.eye(32)
    Hs[1] -= 0.5 * torch.eye(32) * Hs[1].diagonal().mean()  # indefinite, damp x10 fixes
    Hs[3, 7, 7] = -1.0e6  # hopeless
    records = []

    class _Grab(logging.Handler):
        def emit(self, rec):
            records.append(rec.getMessage())

    lg = logging.getLogger(rg.__name__)
    h = _Grab()
    lg.addHandler(h)
    try:
        U_ok = rg._prepare_hinv(Hs[:3].clone(), 0.01)
        tensors["hinv.H_ok"] = Hs[:3].clone()
        tensors["hinv.U_ok"] = U_ok
        meta["hinv_ok_warnings"] = list(records)
        records.clear()
        try:
            rg._prepare_hinv(Hs.clone(), 0.01)
            meta["hinv_fail_message"] = None
        except RuntimeError as exc:
            meta["hinv_fail_message"] = str(exc)
        meta["hinv_fail_warnings"] = list(records)
        tensors["hinv.H_fail"] = Hs.clone()
    finally:
        lg.removeHandler(h)

    # choose_qparams on adversarial small groups (near-ties, constant groups).
    g = torch.Generator().manual_seed(12)
    w = torch.randn(64, 64, generator=g)
    w[0] = 0.0
    w[1] = 1.0
    w[2, :32] = -3.0
    w[3] = torch.linspace(-1, 1, 64)
    w[4] *= 1e-10
    for bits in (2, 4, 8):
        for st in (torch.bfloat16, torch.float16, torch.float32):
            s_st, b_st, s32, b32 = rgrid.choose_qparams(w, bits, "mse", st)
            key = f"qparams.b{bits}.{str(st).split('.')[-1]}"
            tensors[key + ".s32"] = s32
            tensors[key + ".b32"] = b32
    tensors["qparams.w"] = w

    save_file({k: v.contiguous() for k, v in tensors.items()}, str(OUT / "solver_golden.safetensors"))
    (OUT / "solver_golden.json").write_text(json.dumps(meta, indent=1, sort_keys=True))
    print(f"wrote {len(tensors)} tensors")
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
