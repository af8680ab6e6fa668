"""The adaLN modulation projection of redline/host_glue.py on the HIP GEMV.

The reference computes ``modulation(w, te) = linear(silu(te), W_mod)`` and ``norm_out_scale`` in numpy float32 on
fp32 weights (redline/host_glue.py:22-28, :43-48), rows [t, 0]. Here W is the packed b_layout stream of W.T (packed
once on the GPU with ``pack_linear``) and the product is the bandwidth-bound GEMV: y = bf16(Q(silu(te)) @ W.T), with
silu evaluated in fp32, Q the bfp16 activation encoding (blocks of 8 along K) and fp32 accumulation.
"""

import torch

from . import ops


def pack_linear(W):
    """A Linear weight (N, K) (float32 or bf16, any device) -> packed B stream on the GPU."""
    W = torch.as_tensor(W)
    if W.device.type != "cuda":
        W = W.to("cuda")
    return ops.pack_weight(W.contiguous())


def silu_linear(te, w_packed, N):
    """bf16(silu(te) @ W.T) for te (M, K), 1 <= M <= 8, on the GEMV."""
    te = torch.as_tensor(te)
    if te.device.type != "cuda":
        te = te.to("cuda")
    return ops.gemv(te.to(torch.bfloat16).contiguous(), w_packed, N, act="silu")


def modulation(w, te):
    """w: {"modulation.1.weight": packed stream, "modulation.N": N}; te (rows, K) -> (rows, N)
    (redline/host_glue.py:43-44)."""
    return silu_linear(te, w["modulation.1.weight"], w["modulation.N"])


def norm_out_scale(w, te):
    """(redline/host_glue.py:47-48) on the GEMV."""
    return silu_linear(te, w["norm_out.linear.weight"], w["norm_out.N"])
