"""Host adapters of redline/run_glue.py: the fused SwiGLU path's stream adapters and the glue math (silu, rope,
rms_rope).

In the reference, run_glue.swiglu_pack builds the config3 C stream with [gate 64 | proj 64] per 128-column tile and
swiglu_unpack decodes the SwiGLU kernel's output (down-GEMM A tiles, a_layout(., 128, 64)) (redline/run_glue.py:
109-124). On the HIP path the SwiGLU is an epilogue of the up GEMM; these adapters convert between those NPU streams
and the GPU tensors, on the GPU.
"""

import torch

from . import ops


def silu(x):
    return x / (1.0 + torch.exp(-x))


def rope(y, cos, sin):
    """Complex RoPE on adjacent dim pairs: y (n, 128), cos/sin (n, 64) (redline/run_glue.py:27-32)."""
    a, b = y[:, 0::2], y[:, 1::2]
    out = torch.empty_like(y)
    out[:, 0::2], out[:, 1::2] = a * cos - b * sin, a * sin + b * cos
    return out


def rms_rope(x, w, cos, sin):
    """RMSNorm over the last dim (eps 1e-6) * w, then RoPE (redline/run_glue.py:35-37); the fused HIP pass that does
    this for every head of the QKV GEMM's output is ops.qkv_post."""
    return rope(x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w, cos, sin)


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
