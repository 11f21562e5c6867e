"""Host-side API behaviour that needs no GPU: argument validation raises the
reference's exception types before any device work, and the product path
refuses to compute without a HIP device (no CPU fallback)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from mlx_gptq import grid, packing


def test_mode_defaults_and_errors():
    assert grid.mode_defaults("mxfp4") == (32, 4)
    assert grid.mode_defaults("mxfp8") == (32, 8)
    assert grid.mode_defaults("affine") == (64, 4)
    with pytest.raises(ValueError):
        grid.mode_defaults("int3")
    with pytest.raises(ValueError):
        grid._mxfp_max("affine")
    assert grid._E2M1_VALUES[7] == 6.0 and grid.MX_GROUP_SIZE == 32


def test_pack_validation_precedes_device_work():
    with pytest.raises(ValueError):
        packing.pack_q(np.zeros((2, 8), dtype=np.uint8), 3)
    with pytest.raises(AssertionError):
        packing.pack_mxfp4(np.zeros(4, dtype=np.uint8))


def test_rtn_mxfp_validation():
    with pytest.raises(ValueError):
        grid.rtn_quantize_mxfp(torch.zeros(2, 48), "mxfp4")


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the no-GPU behaviour")
def test_no_cpu_fallback_without_gpu():
    with pytest.raises(RuntimeError, match="HIP devices only"):
        grid.rtn_quantize_mxfp(torch.zeros(2, 64), "mxfp4")
    with pytest.raises(RuntimeError, match="HIP devices only"):
        packing.pack_q(np.zeros((2, 8), dtype=np.uint8), 4)


def test_packed_out_validation():
    """solve_gptq's packed_out is checked for shape, dtype, layout, device and
    alignment before any launch (gptq._check_packed), for the pack widths
    pack_q accepts (packing.py:15-26)."""
    from mlx_gptq import gptq

    dev = torch.device("cpu")
    ok = torch.zeros(2, 3, 64 * 4 // 32, dtype=torch.int32)
    gptq._check_packed(ok, (2, 3, 64), 4, dev)
    gptq._check_packed(torch.zeros(2, 3, 16, dtype=torch.int32), (2, 3, 64), 8, dev)
    bad = [torch.zeros(2, 3, 9, dtype=torch.int32),            # wrong width
           torch.zeros(2, 3, 8, dtype=torch.int64),            # wrong dtype
           torch.zeros(2, 3, 16, dtype=torch.int32)[..., ::2]]  # not contiguous
    for b in bad:
        with pytest.raises(ValueError, match="packed_out"):
            gptq._check_packed(b, (2, 3, 64), 4, dev)
    with pytest.raises(ValueError, match="cannot pack"):
        gptq._check_packed(ok, (2, 3, 64), 3, dev)
    with pytest.raises(ValueError, match="packed_out"):
        gptq._check_packed(ok, (2, 3, 64), 4, torch.device("meta"))
