"""CPU oracle for the GPTQ calibration solver -- TEST INFRASTRUCTURE ONLY.

A from-scratch torch-CPU / numpy restatement of the reference algorithm
(mlx_gptq/gptq.py, grid.py, packing.py, artifacts.py:30-39,
capture.py:42-50,68-76 of the reference repository). It reproduces the
reference's op sequence (same torch / LAPACK / numpy calls in the same order)
so that, on the same inputs and the same torch build, it yields the same
bits as the reference.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker (or the timed CPU baseline).
The product (mlx-gptq-mxfp_amd/) never imports it.

Pinning (what fixes each function independently of this restatement):
  grid_ref.choose_mxfp_scale   torch log2/round (library routine) + the
                               closed-form binade thresholds; golden vectors
  grid_ref._e2m1_codes         closed form (RNE on the E2M1 grid); golden vectors
  grid_ref.quantize_mxfp_with_scale  E4M3: torch float8_e4m3fn cast (library);
                               golden vectors
  grid_ref.choose_qparams      brute force over the 21 candidates; golden vectors
  packing_ref.*                known answer (0x76543210, 0xFEDCBA98) + closed form
  hessian_ref.stash_hessian    closed form X^T X vs fp64
  gptq_ref.prepare_hinv        LAPACK uniqueness: U^T U (H + lam I) = I, upper,
                               positive diagonal; escalation on crafted inputs
  gptq_ref.gptq_quantize       golden vectors written by the reference itself
                               (tests/golden/make_golden.py) + the reference's
                               own invariants (tests/test_gptq.py)
"""
