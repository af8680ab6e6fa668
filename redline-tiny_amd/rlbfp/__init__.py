"""rlbfp: the bfp16-weight GEMM path of redline-tiny on MI355X (gfx950), over the C ABI in include/rlbfp.h.

  ops        quantize / dequantize / pack_weight, gemm (fused bias, GELU, SwiGLU, gate*acc + residual,
             re-quantize), gemm_grouped, gemv
  layouts    npu_layouts names (to_bfp16, from_bfp16, pack_b, ...) on the GPU
  forward    forward.py's GEMM call surface: GEMMS, GEMM_KN, v9, NPU, Weights, gemm
  host_glue  the adaLN modulation projection on the GEMV
  run_glue   SwiGLU stream adapters
"""

from . import _lib, ops  # noqa: F401
from ._lib import RLError  # noqa: F401

__version__ = "0.1.0"


def version():
    return _lib.lib().rl_version().decode()
