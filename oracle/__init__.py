"""CPU oracle for the bfp16 GEMM path: TEST INFRASTRUCTURE ONLY.

Only the tests, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import this package, and
only to check results against (or, in the baseline leg, to time the CPU path). The product (``redline-tiny_amd/``)
never imports it and has no CPU fallback.

Modules
  bfp16   the bfp16ebs8 format (encode / decode), the NPU stream layouts and the weight packer, restated in numpy
          from redline/npu_layouts.py, redline/pack_weights.py and redline/forward.py (file:line in each docstring).
  gemm    the CPU emulation of the GEMM path: decode both operands, float64 matmul, fused epilogues, bf16 rounding;
          the adaLN modulation GEMV; the row-RMS-normalised activation generator.
  bfp16_c the same encoder restated a second time in plain C with integer arithmetic (``bfp16_ref.c``), built by
          ``oracle/Makefile``; it cross-checks the numpy encoder and is the fast encoder for large test inputs.

Pinning (what checks each function, so that a plausible mistake fails at least one of them):
  to_bfp16      hand-derived known answers (ties to even, +127 saturation, -128 kept, subnormal block, large spread),
                the C restatement (independent integer algorithm) on random and adversarial inputs, the closed-form
                invariants (|q| of the max-exponent element in [64, 127], decode error <= half a step), and the
                -128 corner where re-encoding a decoded block is not the identity.
  from_bfp16    known answers above, and exactness against float64 products.
  layouts       inverse pairs, and the independent scalar index formulas (forward.py:64-80 and the B-stream formula).
  bf16_round    torch's float32 -> bfloat16 cast (a library routine) on random and tie-heavy inputs.
  gemm / gemv   decoded operands multiplied in float64 vs a brute-force triple loop on tiny shapes, and the epilogue
                formulas against their closed forms (silu(0)=0, gelu odd-part identity, gate 0 -> residual).
"""
