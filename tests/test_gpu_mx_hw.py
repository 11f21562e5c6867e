"""The solver's MXFP element arithmetic on gfx950's scaled MX conversion
instructions (csrc/mx_hw.h), checked on the GPU for every fp32 weight at a
spread of scale exponents against the exact software encoders of
csrc/mgq_common.h (themselves pinned to the reference's threshold chain,
grid.py:82-105, by tests/test_mx4_projection.py, and to torch's float8_e4m3fn
cast by the encoder tests):

- codes and dq of the recurrence's encoders: bit-exact; the NaN-free forms
  (the fast pass and the RTN fallback) bit-exact for every non-NaN n, the
  MXFP4 one as written into one byte of a codes word;
- candidate errors (q - n) used to score scale candidates: bit-exact except
  where n = w / scale is below 2^-126 in magnitude, where both are below it;
- for bf16 weights those errors are exact in bf16 whenever
  2^-126 <= |n| < 512 (MXFP4) or < 16384 (MXFP8), which is what lets the
  candidate objective take them as a single bf16 MFMA operand.

The library is built by build() from tests/native/check_mx_hw.hip.
"""

from __future__ import annotations

import ctypes
import os

import pytest

pytestmark = pytest.mark.gpu

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "libmgq_hwcheck.so")
KINDS = ["mx4 code", "mx4 dq", "mx8 code", "mx8 dq", "mx4 cand err", "mx8 cand err",
         "mx4 err not bf16", "mx8 err not bf16", "mx4 NaN-free byte encode", "mx8 NaN-free encode"]


@pytest.mark.parametrize("e", [-127, -126, -125, -64, -9, -1, 0, 1, 7, 64, 119, 120, 126, 127])
def test_hw_mx_conversions_exhaustive(e):
    import torch

    assert torch.cuda.is_available()
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} missing: run build() first")
    lib = ctypes.CDLL(LIB)
    lib.mgq_hwcheck_mx.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_ulonglong)]
    counts = (ctypes.c_ulonglong * len(KINDS))()
    assert lib.mgq_hwcheck_mx(e, counts) == 0
    bad = {k: int(c) for k, c in zip(KINDS, counts) if c}
    assert not bad, (e, bad)


def test_markstein_division_matches_ieee():
    """div_exact, the correction and range guards that the affine column
    loop's divisions take (err = (w - q) / U[c,c] and the clip scale),
    against IEEE fp32 division, bit for bit: every 64th divisor significand
    against all 2^23 dividend significands (the full 2^46 pairs were checked
    the same way with stride 1), plus random pairs over the exponent range
    on both sides of the guards."""
    import torch

    assert torch.cuda.is_available()
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} missing: run build() first")
    lib = ctypes.CDLL(LIB)
    lib.mgq_hwcheck_div.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_ulonglong)]
    counts = (ctypes.c_ulonglong * 2)()
    assert lib.mgq_hwcheck_div(6, counts) == 0
    assert list(counts) == [0, 0]


def test_scaled_decode_folds_the_scale_exactly():
    """v_cvt_scalef32_pk_f32_fp4 / _fp8 with the E8M0 scale passed in equal
    the decode at scale 1 times the scale, bit for bit, for every byte
    value, byte position and scale 2^-127 .. 2^127: the solver's dq
    (value(code) * scale, grid.py's dequantize) may take the scale in the
    conversion."""
    import torch

    assert torch.cuda.is_available()
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} missing: run build() first")
    lib = ctypes.CDLL(LIB)
    lib.mgq_hwcheck_scaled_decode.argtypes = [ctypes.POINTER(ctypes.c_ulonglong)]
    counts = (ctypes.c_ulonglong * 2)()
    assert lib.mgq_hwcheck_scaled_decode(counts) == 0
    assert (int(counts[0]), int(counts[1])) == (0, 0), (int(counts[0]), int(counts[1]))
