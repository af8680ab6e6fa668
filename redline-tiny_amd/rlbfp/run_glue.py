"""Host adapters of redline/run_glue.py for the fused SwiGLU path.

In the reference, run_glue.swiglu_pack builds the config3 C stream with [gate 64 | proj 64] per 128-column tile and
swiglu_unpack decodes the SwiGLU kernel's output (down-GEMM A tiles, a_layout(., 128, 64)) (redline/run_glue.py:
109-124). On the HIP path the SwiGLU is an epilogue of the up GEMM; these adapters convert between those NPU streams
and the GPU tensors, on the GPU.
"""

import torch

from . import ops


def silu(x):
    return x / (1.0 + torch.exp(-x))


def swiglu_pack(gate, proj):
    """gate / proj (M, F) device tensors -> (C stream bytes in the ATB order with the [gate 64 | proj 64]
    interleave, bfp16-rounded gate, bfp16-rounded proj), like redline/run_glue.py:109-119."""
    M, F = gate.shape
    c = torch.stack([gate.float().reshape(M, F // 64, 64), proj.float().reshape(M, F // 64, 64)], 2).reshape(M, 2 * F)
    packed, deq = ops.quantize(c.contiguous(), order="c_atb", deq=True)
    t = deq.float().reshape(M, F // 64, 2, 64)
    return packed, t[:, :, 0].reshape(M, F), t[:, :, 1].reshape(M, F)


def swiglu_unpack(a_t, M, F):
    """The SwiGLU output as down-GEMM A tiles (a_layout(., 128, 64) bytes) -> (M, F) float32
    (redline/run_glue.py:122-124)."""
    return ops.dequantize(a_t, M, F, order="a_layout")
