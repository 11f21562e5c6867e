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
